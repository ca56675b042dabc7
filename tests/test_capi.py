"""The C-ABI library loads and exports every symbol include/dfssm.h declares; validation paths
that return before any launch behave as documented. No GPU needed."""
import ctypes
import os
import re

import pytest

from dfssm import _C

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(REPO, "include", "dfssm.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(dfssm_\w+)\s*\(", text, re.M)))


def test_header_symbols_exported():
    names = _declared()
    assert len(names) >= 18, names
    lib = ctypes.CDLL(_C.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/dfssm.h but not exported"
    assert set(names) == set(_C.exported_symbols()), "binding and header disagree"


def test_version_and_errors():
    L = _C.lib()
    assert L.dfssm_version() == 7
    assert L.dfssm_error_string(-2).decode().startswith("model dimensions")


def _dims(**kw):
    base = dict(n_layer=48, d_model=2048, d_inner=4096, d_state=128, nheads=64, headdim=64, ngroups=1,
                vocab_size=50288, batch=1, emb_code=1)
    base.update(kw)
    return _C.Dims(*[base[f] for f, _ in _C.Dims._fields_])


@pytest.mark.parametrize("kw,rc", [({}, 0), ({"batch": 4}, 0), ({"batch": 5}, 0), ({"batch": 64}, 0), ({"batch": 65}, -3), ({"batch": 0}, -3),
                                   ({"d_state": 64}, -2), ({"ngroups": 2}, -2), ({"d_model": 2000}, -2),
                                   ({"emb_code": 0}, 0), ({"emb_code": 2}, -2), ({"nheads": 60}, -2),
                                   ({"d_model": 2560, "d_inner": 5120, "nheads": 80}, 0),
                                   ({"vocab_size": 65536}, 0), ({"vocab_size": 65537}, -2)])
def test_check_dims(kw, rc):
    assert _C.lib().dfssm_check_dims(_dims(**kw)) == rc


def test_sizes():
    L = _C.lib()
    assert L.dfssm_tiled_bits_bytes(8512, 2048) == 8512 * 64 * 4
    assert L.dfssm_tiled_bits_bytes(10576, 2560) == 10624 * 80 * 4   # rows padded to 64
    assert L.dfssm_tiled_emb_bytes(50288, 2048) == 50304 * 2048
    assert L.dfssm_tiled_emb_bytes(50288, 4096) == 50304 * 4096   # fp16 rows
    assert L.dfssm_workspace_bytes(_dims()) > 0
    assert L.dfssm_workspace_bytes(_dims(batch=65)) == 0


def test_static_workspace_covers_batch32():
    """DFSSM_STATIC_WORKSPACE_BYTES (include/dfssm.h: 24 MiB) holds the decode workspace of batch
    <= 32 at the 1.3B and 2.7B shapes (dfssm_decode_step_static accepts them) and not of batch 64."""
    text = open(os.path.join(REPO, "include", "dfssm.h")).read()
    m = re.search(r"#define DFSSM_STATIC_WORKSPACE_BYTES \((\d+)u << (\d+)\)", text)
    cap = int(m.group(1)) << int(m.group(2))
    L = _C.lib()
    shapes = ({}, {"n_layer": 64, "d_model": 2560, "d_inner": 5120, "nheads": 80})
    for kw in shapes:
        for B in (1, 4, 5, 17, 32):
            assert 0 < L.dfssm_workspace_bytes(_dims(batch=B, **kw)) <= cap, (kw, B)
        assert L.dfssm_workspace_bytes(_dims(batch=64, **kw)) > cap, kw


def test_null_and_shape_rejections_before_launch():
    L = _C.lib()
    assert L.dfssm_scaffold_gemm(None, None, None, None, 1, 8, 2048, None, None, None) == -1
    assert L.dfssm_scaffold_gemm(16, 16, None, None, 65, 8, 2048, 16, None, None) == -3
    assert L.dfssm_scaffold_gemm(16, 16, None, None, 0, 8, 2048, 16, None, None) == -3
    assert L.dfssm_scaffold_gemm(16, 16, None, None, 1, 8, 1000, 16, None, None) == -2
    assert L.dfssm_scaffold_gemm(8, 16, None, None, 1, 8, 2048, 16, None, None) == -4
    assert L.dfssm_ssm_step(16, 16, 4352, 16, 64, 16, 16, 16, 16, 4096, 1, 64, 64, 64, None) == -2
    assert L.dfssm_tile_bits(None, None, 8, 2048, None) == -1
    assert L.dfssm_layer_step(None, 0, None, None, None, None) == -1
