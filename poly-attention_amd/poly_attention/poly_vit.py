"""PolyViT: drop-in for ``poly_attention/poly_vit.py`` (lucidrains/poly-attention 0.3.6).

An image is cut into non-overlapping patches, each patch (its pixels in patch-row, patch-column,
channel order) is layer-normed, projected to ``dim`` and layer-normed again; a fixed 2-D sine
/ cosine table is added; ``depth`` residual blocks of [poly attention (pre-RMSNorm, not causal),
feed-forward (LayerNorm, Linear, GELU, Linear)] follow, then a LayerNorm, the mean over the
patches and a bias-free linear head (poly_vit.py:65-101; the reference has no class token).

What is forced by interchangeable state dicts and seeded initialisation: the attribute names,
the index layout of ``to_patch_embedding`` (1: LayerNorm, 2: Linear, 3: LayerNorm) and of
each block (``transformer.layers[i]`` = [attention, feed-forward], the feed-forward's 0 / 1 / 3
entries) and the order in which the layers are created.  The GEMMs and norms around the
attention are stock torch (hipBLASLt); each block's attention core runs on the HIP kernels.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.nn import Module, ModuleList

from .n_poly_attention import NPolyAttention
from .poly_attention import Order2PolyAttention


def _two(v):
    return tuple(v) if isinstance(v, tuple) else (v, v)


def posemb_sincos_2d(h: int, w: int, dim: int, temperature: int = 10000,
                     dtype=torch.float32) -> Tensor:
    """[h * w, dim] position table for a row-major h x w patch grid (poly_vit.py:19-30): with
    a quarter of the features per component and frequencies temperature^(-k / (dim/4 - 1)),
    the features are [sin(col f), cos(col f), sin(row f), cos(row f)]."""
    assert dim % 4 == 0, "feature dimension must be multiple of 4 for sincos emb"
    quarter = dim // 4
    # 1 / T^e rather than T^-e: the same roundings as the reference's table
    freqs = 1.0 / (temperature ** (torch.arange(quarter) / (quarter - 1)))
    rows = torch.arange(h).repeat_interleave(w)          # patch index -> grid row
    cols = torch.arange(w).repeat(h)                     # patch index -> grid column
    col_ang = torch.outer(cols.to(freqs.dtype), freqs)
    row_ang = torch.outer(rows.to(freqs.dtype), freqs)
    return torch.cat([col_ang.sin(), col_ang.cos(), row_ang.sin(), row_ang.cos()], dim=1).to(dtype)


def _patches(img: Tensor, ph: int, pw: int) -> Tensor:
    """[b, c, H, W] -> [b, (H/ph)(W/pw), ph * pw * c]: patches in row-major grid order, each
    flattened with the channel fastest, then the column, then the row inside the patch."""
    b, c = img.shape[:2]
    grid = img.unfold(2, ph, ph).unfold(3, pw, pw)        # b, c, gh, gw, ph, pw
    grid = grid.permute(0, 2, 3, 4, 5, 1)                 # b, gh, gw, ph, pw, c
    return grid.reshape(b, grid.shape[1] * grid.shape[2], ph * pw * c)


class _Patchify(Module):
    """Slot 0 of ``to_patch_embedding`` (no parameters): the patch cut of ``_patches``."""

    def __init__(self, ph: int, pw: int):
        super().__init__()
        self.ph, self.pw = ph, pw

    def forward(self, img: Tensor) -> Tensor:
        return _patches(img, self.ph, self.pw)


def FeedForward(dim: int, hidden_dim: int) -> nn.Sequential:
    """LayerNorm -> Linear(dim, hidden) -> GELU -> Linear(hidden, dim) (poly_vit.py:34-40)."""
    return nn.Sequential(nn.LayerNorm(dim), nn.Linear(dim, hidden_dim), nn.GELU(),
                         nn.Linear(hidden_dim, dim))


class Transformer(Module):
    """``depth`` pre-normed residual blocks and a final LayerNorm (poly_vit.py:42-63)."""

    def __init__(self, dim, depth, heads, dim_head, mlp_dim, order=2, use_flash_kernel=None):
        super().__init__()
        self.norm = nn.LayerNorm(dim)
        blocks = []
        for _ in range(depth):  # attention first, then feed-forward: the seeded init order
            if order == 2:
                attn = Order2PolyAttention(dim=dim, heads=heads, dim_head=dim_head, causal=False,
                                           prenorm=True, use_flash_kernel=use_flash_kernel)
            else:
                attn = NPolyAttention(dim=dim, order=order, heads=heads, dim_head=dim_head,
                                      causal=False, prenorm=True)
            blocks.append(ModuleList([attn, FeedForward(dim, mlp_dim)]))
        self.layers = ModuleList(blocks)

    def forward(self, x: Tensor) -> Tensor:
        for block in self.layers:
            attn, ff = block[0], block[1]
            x = x + attn(x)
            x = x + ff(x)
        return self.norm(x)


class PolyViT(Module):
    """Image classifier on poly attention (poly_vit.py:65-101)."""

    def __init__(self, *, image_size, patch_size, num_classes, dim, depth, heads, mlp_dim,
                 channels=3, dim_head=64, order=2, use_flash_kernel=None):
        super().__init__()
        (ih, iw), (ph, pw) = _two(image_size), _two(patch_size)
        assert ih % ph == 0 and iw % pw == 0, 'Image dimensions must be divisible by the patch size.'
        patch_dim = channels * ph * pw
        self.to_patch_embedding = nn.Sequential(_Patchify(ph, pw), nn.LayerNorm(patch_dim),
                                                nn.Linear(patch_dim, dim), nn.LayerNorm(dim))
        # a buffer outside the state dict (the reference's state dict has no position table):
        # it moves with the module, so a forward issues no host-to-device copy and can be
        # captured into a HIP graph; the reference moves it on every call (poly_vit.py:96)
        self.register_buffer("pos_embedding", posemb_sincos_2d(h=ih // ph, w=iw // pw, dim=dim),
                             persistent=False)
        self.transformer = Transformer(dim, depth, heads, dim_head, mlp_dim, order=order,
                                       use_flash_kernel=use_flash_kernel)
        self.linear_head = nn.Linear(dim, num_classes, bias=False)

    def _apply(self, fn, recurse=True):
        # Module casts (.half(), .to(torch.bfloat16), ...) must not round the position table:
        # the reference keeps it in fp32 and casts it at each forward (poly_vit.py:96), so that
        # e.g. model.half().float() still adds the exact table.  Only the device follows fn.
        table = self.pos_embedding
        out = super()._apply(fn, recurse)
        self.pos_embedding = table.to(device=self.pos_embedding.device, dtype=torch.float32)
        return out

    def forward(self, img: Tensor) -> Tensor:
        tokens = self.to_patch_embedding(img)
        tokens = tokens + self.pos_embedding.to(img.device, dtype=img.dtype)
        tokens = self.transformer(tokens)
        return self.linear_head(tokens.mean(dim=1))


# the reference's helper names (poly_vit.py:13-17)
def pair(t):
    return _two(t)


def divisible_by(num, den) -> bool:
    return num % den == 0
