"""MI355X-native DF-SSM decode step: .dfssm format, HIP kernel bindings and host runtime."""
from .format import (DFSSMConfig, DFSSMWeights, DFSSMFormatError, read_dfssm, write_dfssm,
                     expected_size, layer_bytes, pack_sign_bits, unpack_sign_bits,
                     EMB_F16, EMB_I8, NORM_F32, NORM_F16, LORA_RANK, D_CONV)

__version__ = "0.1.0"
