"""fp8 e4m3 weight quantization and the fp8-weight FFN (oracle), CPU.

TEST INFRASTRUCTURE ONLY (see the package docstring).

The reference has no fp8 path: its FFN is FeedForward("gelu-approximate")
(投机采样/wam-p0-worktree/wan_va/modules/model.py:790, Linear -> GELU(tanh)
-> Linear) followed by the gated residual (model.py:792-793).  The fp8 variant
of the FFN unit replaces each weight W [N, K] by per-output-channel e4m3
values with one fp32 scale per row:

  scale[n] = max_k |W[n, k]| / 448      (1 for an all-zero row)
  q[n, k]  = e4m3fn(W[n, k] / scale[n])  round to nearest even, |q| <= 448

and computes with W' = q * scale (bf16 activations, fp32 accumulation).  The
rounding is torch's float8_e4m3fn cast (OCP E4M3: 4 exponent bits, bias 7, 3
mantissa bits, max 448, no infinities); tests/test_oracle.py pins it against
hand-decoded e4m3 values.
"""
import torch
import torch.nn.functional as F

E4M3 = torch.float8_e4m3fn
E4M3_MAX = 448.0


def quantize_rows(w):
    """w [N, K] (bf16 or fp32) -> (q [N, K] float8_e4m3fn, scale [N] fp32)."""
    wf = w.float()
    amax = wf.abs().amax(dim=1)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (wf / scale[:, None]).to(E4M3)
    return q, scale


def dequantize_rows(q, scale):
    return q.float() * scale[:, None]


def e4m3_decode(byte):
    """Value of one OCP e4m3fn byte, decoded from its bit fields."""
    s = -1.0 if byte & 0x80 else 1.0
    e = (byte >> 3) & 0xF
    m = byte & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def ffn_gated(x, w1, b1, w2, b2, residual, gate):
    """residual + (GELU_tanh(x W1^T + b1) W2^T + b2) * gate, all fp32 (the
    oracle's FFN unit; model.py:790-793 with the bf16 roundings removed)."""
    h = F.gelu(x.float() @ w1.float().t() + b1.float(), approximate="tanh")
    return residual.float() + (h @ w2.float().t() + b2.float()) * gate.float()
