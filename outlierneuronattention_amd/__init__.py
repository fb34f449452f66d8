"""MI355X-native HOFA hybrid attention (outlier softmax + inlier GLA).

Drop-in for the reference's attention path: the module classes, the op
functions (``chunk_gla_inlier_fwd``, ``exact_attention``, ``fused_hofa_decode``)
and the cache / state layout keep the reference's names and meaning; the
arithmetic runs in hand-written gfx950 HIP kernels behind the C ABI of
``include/hofa.h`` (``libhofa.so``).
"""
from .hofa_decode import fused_hofa_decode  # noqa: F401

__all__ = ["fused_hofa_decode"]
