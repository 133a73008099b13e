"""Weight-layout helpers for per-head projections.

`interleave_qkv` and `interleave_kv` keep the reference's layouts (the precompute dict
entries are part of its observable API, `triangle_ops/_common/layouts.py:11-31`).
`qkv_head_major` is the layout the gfx950 kernels load: per head, the rows of WQ^T, WK^T
and WV^T, so a lane reads 8 consecutive input channels of one output feature (16 bytes).
"""

import torch


def interleave_qkv(WQ: torch.Tensor, WK: torch.Tensor, WV: torch.Tensor, H: int, D: int) -> torch.Tensor:
    """(C, H*D) x 3 -> (C, 3*H*D); columns [3hD, 3(h+1)D) hold [Q_h | K_h | V_h] (x @ W convention)."""
    C = WQ.shape[0]
    assert WQ.shape == WK.shape == WV.shape == (C, H * D)
    per_head = [t.reshape(C, H, 1, D) for t in (WQ, WK, WV)]
    return torch.cat(per_head, dim=2).reshape(C, 3 * H * D).contiguous()


def interleave_kv(WK: torch.Tensor, WV: torch.Tensor, H: int, D: int) -> torch.Tensor:
    """(C, H*D) x 2 -> (C, 2*H*D); per head the 2D columns alternate K[d], V[d] (feature interleave)."""
    C = WK.shape[0]
    assert WK.shape == WV.shape == (C, H * D)
    return torch.stack((WK.reshape(C, H, D), WV.reshape(C, H, D)), dim=3).reshape(C, 2 * H * D).contiguous()


def qkv_head_major(WQ: torch.Tensor, WK: torch.Tensor, WV: torch.Tensor, H: int, D: int) -> torch.Tensor:
    """(C, H*D) x 3 -> (H, 3, D, C): per head, the rows of WQ^T, WK^T, WV^T."""
    C = WQ.shape[0]
    assert WQ.shape == WK.shape == WV.shape == (C, H * D)
    w = torch.stack((WQ.reshape(C, H, D), WK.reshape(C, H, D), WV.reshape(C, H, D)), dim=0)  # (3, C, H, D)
    return w.permute(2, 0, 3, 1).contiguous()
