"""deciax_amd — MI355X-native decision-prefill path for deciax.

`load(...).decide / decide_batch` as in the reference (src/deciax/__init__.py,
src/deciax/decider.py), served by hand-written gfx950 HIP kernels behind the C
ABI of `include/deciax_hip.h` (`libdeciax_hip.so`, built by
`python -m deciax_amd.build`).
"""

from deciax_amd.decider import Decider, load

__all__ = ["Decider", "load"]
__version__ = "0.1.0"
