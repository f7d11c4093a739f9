"""MI355X-native (gfx950) DeepSeek sparse-attention (DSA) path for torchtitan.

Drop-in for the reference's ``npu_dsa`` / ``npu_smla`` converters and the torch_npu DSA
ops they call.  Compute runs only in the HIP library ``libdsa_mi355x.so`` (C ABI in
``include/dsa_mi355x.h``); Python here is plumbing: ctypes calls, autograd wrappers and
the ModelConverter registry.
"""

from ._lib import DSAError, load_library  # noqa: F401

__version__ = "0.1.0"
