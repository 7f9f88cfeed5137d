"""MI355X (gfx950) HIP backend for inference_c's tensor-ops hot path.

The product is the C-ABI library libinference_sdk_hip.so built from csrc/
(declarations in include/*.h at the repository root). This package only
locates and binds it: see sdk.py.
"""
from .sdk import (COMPUTE_SLOTS, DEVICE, HOST, LIB_PATH, ComputeBackend, Sdk, SdkError, Tensor, TensorView,  # noqa: F401
                  declared_functions, load_library)
