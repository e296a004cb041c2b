"""MI355X-native PairFormer hot path for DeepFold3 (HIP kernels for gfx950).

The package directory name contains a hyphen, so it is imported under the
alias ``deepfold3_dev_amd`` (see ``load_package`` in ``__graft_entry__.py``).

Layout:
    csrc/            HIP kernels and the C ABI (built into libpairformer_hip.so)
    _lib.py          ctypes binding of the C ABI
    kernels.py       functional ops with the reference kernel layer's signatures
    ops.py           TriangleMulOutgoing / TriangleMulIncoming
    attention.py     GridSelfAttention / SingleAttention
    primitives.py    LayerNorm, LinearNoBias, TransitionBlock
    evoformer.py     PairFormerBlock and the trunk loop
    weights.py       deterministic synthetic weights and inputs
"""

from . import kernel_census  # noqa: F401
from .config import OptimConfig  # noqa: F401
from .inference_guard import InferenceOnlyKernelError, NotActive  # noqa: F401

__version__ = "0.1.0"
