"""poly_attention -- MI355X-native drop-in for lucidrains/poly-attention 0.3.6.

Public names as the reference's ``poly_attention/__init__.py:1-7``.  The attention core runs
in libpolyattn.so (hand-written HIP kernels for gfx950) on GPU tensors.  One addition:
``StaticCache``, a fixed-capacity KV cache for decode loops captured into a HIP graph.
"""

from poly_attention.poly_attention import Order2PolyAttention
from poly_attention.n_poly_attention import NPolyAttention

PolyAttention = Order2PolyAttention

from poly_attention.poly_vit import PolyViT  # noqa: E402
from poly_attention.poly_transformer import PolyTransformer  # noqa: E402
from poly_attention._cache import StaticCache  # noqa: E402

__version__ = "0.3.6"
