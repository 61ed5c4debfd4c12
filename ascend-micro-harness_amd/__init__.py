"""MI355X-native TurboQuant TQ4 quantised-KV hot path.

The package directory is not an importable identifier; load it with
``__graft_entry__.package()`` (importlib, registered as
``ascend_micro_harness_amd``). The compute lives in libtq4.so (HIP kernels
for gfx950 behind the C ABI of include/tq4.h); ``tq4`` is the host mirror and
``torch_ops`` registers it as the ``torch.ops.tq4`` operators.
"""
from .tq4 import *  # noqa: F401,F403
from .tq4 import __all__  # noqa: F401
from . import torch_ops  # noqa: F401  (registers torch.ops.tq4.*)
