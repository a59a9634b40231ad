"""mamba_int: MI355X-native integer Mamba inference path (spec mi-spec-2).

Host side in Python on PyTorch-ROCm; compute in libmamba_int.so (gfx950 HIP
kernels behind the C ABI of include/mamba_int.h).
"""
from .params import (ModelDims, ModelParams, LayerParams, SSDLayerParams, init_random_params,  # noqa: F401
                     pack_ternary, ssd_decay_table, unpack_ternary)

SPEC_VERSION = "mi-spec-2"
