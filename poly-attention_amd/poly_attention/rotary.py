"""Rotary position embedding with the interface the reference uses from
``rotary-embedding-torch>=0.8.9`` (pyproject.toml:29): ``RotaryEmbedding(dim)`` called on
positions, ``rotate_queries_or_keys``, ``rotate_queries_with_cached_keys`` and the module
function ``apply_rotary_emb`` (call sites: poly_attention.py:14,202,277,303-304;
n_poly_attention.py:118,191,224-229; train_enwik8.py:143,160-161).

Restated from the published algorithm (RoFormer, Su et al. 2021) in the layout that package
uses: frequencies ``theta ** (-2k / dim)`` repeated per pair, interleaved pairs
``(x[2k], x[2k+1])`` rotated by ``pos * freq_k``, the frequency table held in a parameter
named ``freqs`` so that state-dict keys match, and ``apply_rotary_emb`` using the last
``seq_len`` rows of the frequency table.  RoPE runs before the kernel boundary (plain torch).
"""

from __future__ import annotations

import torch
from torch import Tensor, nn


def rotate_half(x: Tensor) -> Tensor:
    """(x0, x1, x2, x3, ...) -> (-x1, x0, -x3, x2, ...)"""
    x = x.unflatten(-1, (-1, 2))
    x1, x2 = x.unbind(dim=-1)
    return torch.stack((-x2, x1), dim=-1).flatten(-2)


def apply_rotary_emb(freqs: Tensor, t: Tensor, start_index: int = 0, scale: float = 1.0,
                     seq_dim: int = -2, freqs_seq_dim: int | None = None) -> Tensor:
    dtype = t.dtype
    if freqs_seq_dim is None and (freqs.ndim == 2 or t.ndim == 3):
        freqs_seq_dim = 0
    if t.ndim == 3 or freqs_seq_dim is not None:
        seq_len = t.shape[seq_dim]
        freqs = freqs.narrow(freqs_seq_dim, freqs.shape[freqs_seq_dim] - seq_len, seq_len)
    rot_dim = freqs.shape[-1]
    end_index = start_index + rot_dim
    assert rot_dim <= t.shape[-1], (
        f"feature dimension {t.shape[-1]} is not of sufficient size to rotate in all the "
        f"positions {rot_dim}"
    )
    t_left = t[..., :start_index]
    t_middle = t[..., start_index:end_index]
    t_right = t[..., end_index:]
    t_middle = (t_middle * freqs.cos() * scale) + (rotate_half(t_middle) * freqs.sin() * scale)
    return torch.cat((t_left, t_middle, t_right), dim=-1).type(dtype)


class RotaryEmbedding(nn.Module):
    def __init__(self, dim: int, theta: float = 10000.0, interpolate_factor: float = 1.0,
                 learned_freq: bool = False, cache_if_possible: bool = True,
                 cache_max_seq_len: int = 8192):
        super().__init__()
        freqs = 1.0 / (theta ** (torch.arange(0, dim, 2)[: (dim // 2)].float() / dim))
        self.freqs = nn.Parameter(freqs, requires_grad=learned_freq)
        self.learned_freq = learned_freq
        self.interpolate_factor = interpolate_factor
        self.default_seq_dim = -2
        self.cache_if_possible = cache_if_possible
        self.cache_max_seq_len = cache_max_seq_len
        self.register_buffer("dummy", torch.tensor(0), persistent=False)

    @property
    def device(self):
        return self.dummy.device

    def get_seq_pos(self, seq_len: int, device, dtype, offset: int = 0) -> Tensor:
        return (torch.arange(seq_len, device=device, dtype=dtype) + offset) / self.interpolate_factor

    def forward(self, t: Tensor, seq_len: int | None = None, offset: int = 0) -> Tensor:
        freqs = self.freqs
        freqs = t.type(freqs.dtype)[..., None] * freqs
        return freqs.repeat_interleave(2, dim=-1)

    def rotate_queries_or_keys(self, t: Tensor, seq_dim: int | None = None, offset: int = 0,
                               scale: float | None = None) -> Tensor:
        seq_dim = self.default_seq_dim if seq_dim is None else seq_dim
        device, dtype, seq_len = t.device, t.dtype, t.shape[seq_dim]
        seq = self.get_seq_pos(seq_len, device=device, dtype=dtype, offset=offset)
        freqs = self.forward(seq, seq_len=seq_len, offset=offset)
        if seq_dim == -3:
            freqs = freqs[:, None, :]
        return apply_rotary_emb(freqs, t, scale=1.0 if scale is None else scale, seq_dim=seq_dim)

    def rotate_queries_with_cached_keys(self, q: Tensor, k: Tensor, seq_dim: int | None = None,
                                        offset: int = 0):
        seq_dim = self.default_seq_dim if seq_dim is None else seq_dim
        q_len, k_len = q.shape[seq_dim], k.shape[seq_dim]
        assert q_len <= k_len
        rotated_q = self.rotate_queries_or_keys(q, seq_dim=seq_dim, offset=k_len - q_len + offset)
        rotated_k = self.rotate_queries_or_keys(k, seq_dim=seq_dim, offset=offset)
        return rotated_q.type(q.dtype), rotated_k.type(k.dtype)
