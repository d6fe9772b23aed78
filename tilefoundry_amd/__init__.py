"""MI355X-native (gfx950) Qwen3 decode step: HIP kernels behind a C ABI, driven
from PyTorch-ROCm.  ``tilefoundry_amd.qwen3`` holds the engine, the runtime twin
and the weight handling; ``csrc/`` holds the kernels; ``include/tf_decode.h`` the ABI."""

__all__ = ["qwen3"]
