"""Built-in HIP implementations; importing this package registers them.

Mirrors fp8_training/fp8_bench/impls/__init__.py of xuOAO/practice_cuda.
"""
from . import hip_per_block  # noqa: F401
from . import hip_per_channel  # noqa: F401
from . import hip_per_tensor  # noqa: F401
