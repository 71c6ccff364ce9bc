"""fp8 e4m3 weight quantization and the fp8-weight FFN (oracle), CPU.

TEST INFRASTRUCTURE ONLY (see the package docstring).

The reference has no fp8 path: its FFN is FeedForward("gelu-approximate")
(投机采样/wam-p0-worktree/wan_va/modules/model.py:790, Linear -> GELU(tanh)
-> Linear) followed by the gated residual (model.py:792-793).  The fp8 variant
of the FFN unit replaces each weight W [N, K] by per-output-channel e4m3
values with one fp32 scale per row:

  scale[n] = max_k |W[n, k]| / 448      (1 for an all-zero row)
  q[n, k]  = e4m3fn(W[n, k] * f[n])      round to nearest even, |q| <= 448
  f[n]     = 448 / max_k |W[n, k]|       (fp32; 1 for an all-zero row)

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
    # true fp32 divisions by tensors (a Python scalar operand may be applied
    # through a reciprocal, which rounds twice)
    c448 = torch.full_like(amax, E4M3_MAX)
    scale = torch.where(amax > 0, amax / c448, torch.ones_like(amax))
    f = torch.where(amax > 0, c448 / amax, torch.ones_like(amax))
    q = (wf * f[:, None]).to(E4M3)
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


def mx_exponent(amax):
    """e8m0 exponent X of an MX block (OCP MX: 32 e4m3 values sharing one
    power-of-two scale 2^X) whose largest magnitude is amax: the smallest X
    with amax <= 448 * 2^X, floored at -127.  amax float32 tensor, >= 0."""
    m, e = torch.frexp(amax.double())        # amax = m * 2^e, m in [0.5, 1)
    x = (e - 1 - 8).to(torch.int32)          # amax = (2m) 2^(e-1); 448 = 1.75 * 2^8
    x = torch.where(2 * m > 1.75, x + 1, x)  # 2m > 1.75: the next power
    x = torch.where(amax > 0, x, torch.full_like(x, -127))
    return x.clamp(min=-127)


def quantize_mx32(y):
    """y [M, N] (N a multiple of 32) -> (q float8_e4m3fn [M, N], e uint8
    [M, N / 32]) with e = X + 127 per 32-column block and q = e4m3(y * 2^-X),
    round to nearest even (the scaled values stay within +-448)."""
    yf = y.float()
    M, N = yf.shape
    blk = yf.reshape(M, N // 32, 32)
    X = mx_exponent(blk.abs().amax(dim=2))
    q = (blk * torch.pow(2.0, -X.double()).float()[..., None]).reshape(M, N).to(E4M3)
    return q, (X + 127).to(torch.uint8)


def dequantize_mx32(q, e):
    M, N = q.shape
    X = e.to(torch.int32) - 127
    return (q.float().reshape(M, N // 32, 32) * torch.pow(2.0, X.double()).float()[..., None]).reshape(M, N)
