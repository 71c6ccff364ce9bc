"""3D RoPE grid ids and frequencies (oracle).

get_mesh_id follows 投机采样/wam-p0-worktree/wan_va/utils/utils.py:33-53 and
rope_freqs follows WanRotaryPosEmbed, 投机采样/wam-p0-worktree/wan_va/modules/model.py:243-286:
head_dim 128 splits into f/h/w dims 44/42/42, i.e. 22 + 21 + 21 = 64 complex
pairs, base frequencies 1 / theta^(2k / dim) in float64, angles grid * base,
cast to float32, then polar(1, angle) as complex64.
"""
import torch


def get_mesh_id(f, h, w, t=0, f_w=1, f_shift=0, action=False):
    """[4, f*h*w] float ids (frame, row, col, t) in (f, h, w) raster order."""
    f_idx = torch.arange(f_shift, f + f_shift) * f_w
    ff, hh, ww = torch.meshgrid(f_idx, torch.arange(h), torch.arange(w), indexing="ij")
    if action:
        ff = ff + (torch.ones([h]).cumsum(0) / (h + 1)).view(1, -1, 1)
        hh = torch.full_like(hh, -1)
        ww = torch.full_like(ww, -1)
    grid = torch.stack([ff.flatten().to(torch.float32), hh.flatten().to(torch.float32),
                        ww.flatten().to(torch.float32)])
    return torch.cat([grid, torch.full_like(grid[:1], t)], dim=0)


def base_freqs(head_dim=128, theta=10000.0):
    f_dim = head_dim - 2 * (head_dim // 3)
    h_dim = w_dim = head_dim // 3

    def one(dim):
        return 1.0 / (theta ** (torch.arange(0, dim, 2)[: dim // 2].double() / dim))
    return one(f_dim), one(h_dim), one(w_dim)


def rope_freqs(grid_ids, head_dim=128, theta=10000.0):
    """grid_ids [B, >=3, L] -> complex64 [B, L, 1, head_dim/2] (model.py:1077-1078)."""
    fb, hb, wb = base_freqs(head_dim, theta)
    g = grid_ids.double()
    ang = torch.cat([g[:, 0, :, None] * fb, g[:, 1, :, None] * hb, g[:, 2, :, None] * wb], dim=-1)
    ang = ang.float()
    return torch.polar(torch.ones_like(ang), ang)[:, :, None]
