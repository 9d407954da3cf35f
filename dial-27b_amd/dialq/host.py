"""The host operator layer (C++ above the C ABI: QuantLinear, linear_no_bias,
TextLinear, W8A16Linear, GgufMatMul, forward_worker_gguf and the mode gates),
imported from dial-27b_amd/lib/dialq_host*.so.

torch, when installed, is imported first so that the module's HIP runtime
dependency resolves to the one torch already loaded (one runtime per
process)."""
import os
import sys

try:
    import torch  # noqa: F401
except ImportError:
    pass

_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib")
if _LIB not in sys.path:
    sys.path.insert(0, _LIB)

from dialq_host import *  # noqa: E402,F401,F403
