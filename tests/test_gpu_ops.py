"""GPU parity of the single operators against the C oracle (same seeded inputs).

Scaffold accumulators and the RMSNorm/quantizer outputs must be bit-exact; the conv + SSM
recurrence is compared after 128 steps with max|d| / max|ref| <= 1e-3 (fp32 state), the
north-star tolerance for the state.
"""
import numpy as np
import pytest
import torch

from dfssm import ops
from dfssm.format import unpack_sign_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _h(a):  # numpy fp16 -> torch fp16 on the GPU
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV).view(torch.float16)


def _np16(t):
    return t.cpu().view(torch.int16).numpy().view(np.float16)


def _tiled(bits_np, N, K):
    return ops.tile_bits(torch.from_numpy(bits_np.view(np.int32)).to(DEV), N, K)


# N picks 16, 32 or 64 output rows per matrix-core workgroup (N <= 4096, <= 8192, above)
@pytest.mark.parametrize("N,K", [(8512, 2048), (2048, 4096), (10576, 2560), (2048, 5120), (2320, 512), (6144, 1024)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 16, 32, 64])
def test_scaffold_acc_bit_exact(N, K, M):
    """Config 1: in_proj 2048->8512, out_proj 4096->2048 (+2.7B and tiny shapes), int8 ~N(0,40)."""
    print(f"scaffold N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng([1, N, K, M])
    bits = rng.integers(0, 2 ** 32, (N, K // 32), dtype=np.uint32)
    q = np.clip(np.rint(rng.normal(0, 40, (M, K))), -127, 127).astype(np.int8)
    xs = rng.uniform(0.01, 0.05, M).astype(np.float16)
    ws = rng.uniform(0.01, 0.05, N).astype(np.float16)
    acc, y = ops.scaffold_gemm(_tiled(bits, N, K), torch.from_numpy(q).to(DEV), N, _h(xs), _h(ws), want_y=True)
    ref = O.scaffold_acc(bits, q)
    np.testing.assert_array_equal(acc.cpu().numpy(), ref)
    yref = O.dequant_lora(ref, xs, ws, np.zeros((M, 16), np.float16), np.zeros((N, 16), np.int8),
                          np.zeros(N, np.float16))
    np.testing.assert_array_equal(_np16(y).view(np.uint16), yref.view(np.uint16))


@pytest.mark.parametrize("M", [1, 4, 32])
def test_scaffold_extremes(M):
    """All +127 / all -128 activations against all-set / all-clear / random bits: +-K*127, etc."""
    N, K = 192, 2048
    rng = np.random.default_rng(7)
    bits = np.concatenate([np.full((64, K // 32), 0xFFFFFFFF, np.uint32), np.zeros((64, K // 32), np.uint32),
                           rng.integers(0, 2 ** 32, (64, K // 32), dtype=np.uint32)])
    q = np.where(np.arange(M)[:, None] % 2 == 0, 127, -128).astype(np.int8).repeat(K, axis=1).reshape(M, K)
    acc = ops.scaffold_gemm(_tiled(bits, N, K), torch.from_numpy(q).to(DEV), N).cpu().numpy()
    ref = q.astype(np.int64) @ unpack_sign_bits(bits).astype(np.int64).T
    np.testing.assert_array_equal(acc, ref)
    assert acc[0, 0] == 127 * K and acc[0, 64] == -127 * K


@pytest.mark.parametrize("K", [512, 2048, 4096, 5120])
@pytest.mark.parametrize("scale", [1.0, 1e-3, 300.0])
def test_rmsnorm_quantize_bit_exact(K, scale):
    M = 4
    rng = np.random.default_rng([2, K, int(scale * 1000)])
    x = (rng.normal(0, 1, (M, K)) * scale).astype(np.float16)
    x[1, :] = 0                      # all-zero row: amax clamps to 1e-4
    x[2, ::7] = np.float16(scale * 9)  # outliers
    w = (1 + rng.uniform(-0.1, 0.1, K)).astype(np.float32)
    xn, q, s = ops.rmsnorm_quantize(_h(x), torch.from_numpy(w).to(DEV))
    xn_ref = O.rmsnorm(x, w)
    q_ref, s_ref = O.quantize(xn_ref)
    np.testing.assert_array_equal(_np16(xn).view(np.uint16), xn_ref.view(np.uint16))
    np.testing.assert_array_equal(_np16(s).view(np.uint16), s_ref.view(np.uint16))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("B", [1, 32])
def test_conv_ssm_128_steps(B):
    """Config 2: 64 heads x 64, d_state 128, conv channels 4352, 128 sequential steps."""
    H, P, N = 64, 64, 128
    DI = H * P
    C = DI + 2 * N
    steps = 128
    print(f"conv+ssm B={B}", flush=True)
    rng = np.random.default_rng([3, B])
    conv0 = rng.normal(0, 1, (B, C, 3)).astype(np.float16)
    conv_w = rng.normal(0, 0.5, (C, 4)).astype(np.float16)
    conv_b = rng.normal(0, 0.1, C).astype(np.float16)
    A_log = rng.uniform(0, np.log(16), H).astype(np.float32)
    Dp = np.ones(H, np.float32)
    dt_bias = np.zeros(H, np.float32)
    xbc_seq = rng.normal(0, 1, (steps, B, C)).astype(np.float16)
    dt_seq = rng.normal(-2, 1, (steps, B, H)).astype(np.float16)

    g_conv = _h(conv0)
    g_h = torch.zeros(B, H, P, N, dtype=torch.float32, device=DEV)
    g_y = torch.empty(B, DI, dtype=torch.float16, device=DEV)
    tw, tb = _h(conv_w), _h(conv_b)
    tA, tD, tdb = (torch.from_numpy(a).to(DEV) for a in (A_log, Dp, dt_bias))
    r_conv = conv0.copy()
    r_h = np.zeros((B, H, P, N), np.float32)
    ys = []
    for t in range(steps):
        gx = _h(xbc_seq[t])
        ops.conv_step(g_conv, gx, tw, tb)
        ops.ssm_step(g_h, gx, _h(dt_seq[t]), tdb, tA, tD, g_y)
        rx = xbc_seq[t].copy()
        O.conv_step(r_conv, rx, conv_w, conv_b)
        r_y = O.ssm_step(r_h, rx, dt_seq[t], dt_bias, A_log, Dp)
        if t in (0, steps - 1):
            ys.append((_np16(g_y).astype(np.float32), r_y.astype(np.float32)))
    gh = g_h.cpu().numpy()
    rel = np.abs(gh - r_h).max() / np.abs(r_h).max()
    print(f"B={B} state max rel err {rel:.3e}, bit-exact {np.array_equal(gh, r_h)}")
    assert rel <= 1e-3
    # the state update uses only correctly rounded elementwise operations on identical inputs,
    # so it is in fact bit-exact
    np.testing.assert_array_equal(gh, r_h)
    np.testing.assert_array_equal(_np16(g_conv).view(np.uint16), r_conv.view(np.uint16))
    for gy, ry in ys:
        assert np.abs(gy - ry).max() <= 1e-3 * np.abs(ry).max() + 1e-3
