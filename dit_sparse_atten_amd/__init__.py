"""MI355X-native block-sparse self-attention hot path for Wan video DiTs.

Drop-in counterpart of the reference study's ``attention_backends`` package
(yangshuo1230/DiT_Sparse_Atten): the same ``dense`` / ``sparse`` /
``flex_reuse`` backends and Wan attention-processor call signature, computed by
hand-written gfx950 HIP kernels in ``libdsa.so`` behind a C-ABI.
"""

__version__ = "0.1.0"
