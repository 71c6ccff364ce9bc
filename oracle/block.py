"""WanTransformerBlock.forward restated on the CPU (the oracle).

Follows 投机采样/wam-p0-worktree/wan_va/modules/model.py:
  modulation          :751-759  mod = scale_shift_table[None] + temb.float();
                                 chunk order shift, scale, gate, c_shift, c_scale, c_gate
  norm1 + modulate    :761-763  bf16(LN32(x) * (1 + scale) + shift)
  attn1               :595-691  to_q/k/v, RMSNorm over the full row (norm_q/norm_k),
                                 unflatten to heads, RoPE in float64 (:614-623),
                                 original KV cache / candidate rows (:624-686),
                                 SDPA (:37-40), to_out[0]
  gated residual      :771-772  bf16(x.float() + attn * gate)
  norm2               :775-776  FP32LayerNorm(affine) -> bf16
  attn2               :777-782  q from norm2, k/v from the context, no RoPE, no cache
  cross residual      :783      x + attn (a bf16 add)
  norm3 + modulate    :786-788
  ffn                 :790      Linear -> GELU(tanh) -> Dropout(0) -> Linear
  final residual      :792-793  bf16(x.float() + ff.float() * c_gate)
diffusers is not installed; its FP32LayerNorm is F.layer_norm on float32 input
(cast back to the input dtype) and FeedForward("gelu-approximate") is
Linear + F.gelu(approximate="tanh") + Dropout + Linear.

dtype=torch.float32 gives the fp32 oracle (every tensor fp32; RoPE still in
float64).  dtype=torch.bfloat16 emulates the reference's own bf16 run: weights
and activations bf16 except scale_shift_table and norm2 (fp32, the model's
_keep_in_fp32_modules, model.py:809-821), rounding at the same points.
"""
import torch
import torch.nn.functional as F

from . import kvcache

FP32_KEYS = ("scale_shift_table", "norm2.weight", "norm2.bias")


def apply_rope(x, freqs):
    """model.py:614-621: complex rotation of (2j, 2j+1) pairs in float64."""
    xc = torch.view_as_complex(x.to(torch.float64).reshape(*x.shape[:3], -1, 2))
    return torch.view_as_real(xc * freqs).flatten(3).to(x.dtype)


def sdpa(q, k, v):
    """custom_sdpa (model.py:37-40): q/k/v [B, L, H, hd], non-causal."""
    out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    return out.transpose(1, 2)


def _params(p, dtype):
    return {k: (v.float() if k in FP32_KEYS else v.to(dtype)) for k, v in p.items()}


def attention(P, prefix, q_in, kv_in, rotary_emb, heads, eps_q, eps_k, cache=None,
              update_cache=0, candidate_rows=None, evict_order="stable", keep=None, name=None):
    """WanAttention.forward (model.py:595-691), original cache mode.  With `keep`,
    records the intermediates `{name}_q_linear`, `_k_linear`, `_v`, `_q_norm`,
    `_k_norm`, `_q_rope` and `_k_rope` (or `_q` and `_k` without RoPE),
    `_attention`, `_out` (the reference's
    debug names, optimized/csrc/whole_layer.cu:1203-1209)."""
    g = lambda n: P[f"{prefix}.{n}"]
    rec = (lambda n, t: keep.__setitem__(f"{name}_{n}", t)) if keep is not None else (lambda n, t: None)
    D = q_in.shape[-1]
    q = F.linear(q_in, g("to_q.weight"), g("to_q.bias"))
    k = F.linear(kv_in, g("to_k.weight"), g("to_k.bias"))
    v = F.linear(kv_in, g("to_v.weight"), g("to_v.bias"))
    rec("q_linear", q)
    rec("k_linear", k)
    rec("v", v)
    q = F.rms_norm(q, (D,), g("norm_q.weight"), eps_q).unflatten(2, (heads, -1))
    k = F.rms_norm(k, (D,), g("norm_k.weight"), eps_k).unflatten(2, (heads, -1))
    rec("q_norm", q)
    rec("k_norm", k)
    v = v.unflatten(2, (heads, -1))
    if rotary_emb is not None:
        q = apply_rope(q, rotary_emb)
        k = apply_rope(k, rotary_emb)
        rec("q_rope", q)
        rec("k_rope", k)
    else:
        rec("q", q)  # the reference names the unrotated (cross) q/k `cross_q`, `cross_k`
        rec("k", k)
    if candidate_rows is not None:
        if update_cache != 0 or cache is None:
            raise ValueError("candidate verification requires existing read-only KV")
        valid = kvcache.valid_slots(cache)
        hk, hv = cache["k"][:, valid], cache["v"][:, valid]
        rows = candidate_rows
        if (rows.ndim != 1 or rows.numel() != q.shape[0] or rows.dtype != torch.long
                or not bool(((rows >= 0) & (rows < hk.shape[0])).all())):
            raise ValueError("invalid candidate_cache_rows for this KV cache")
        sk = hk.index_select(0, rows).to(k.dtype)
        sv = hv.index_select(0, rows).to(v.dtype)
        out = sdpa(q, torch.cat((sk, k), 1), torch.cat((sv, v), 1))
    else:
        slots = None
        if cache is not None:
            slots = kvcache.update_cache(cache, k, v, is_pred=(update_cache == 1), order=evict_order)
            valid = kvcache.valid_slots(cache)
            k = cache["k"][:, valid].to(q.dtype)
            v = cache["v"][:, valid].to(q.dtype)
        out = sdpa(q, k, v)
        if update_cache == 0 and cache is not None:
            kvcache.restore_cache(cache, slots)
    out = out.flatten(2, 3).type_as(q)
    rec("attention", out)
    out = F.linear(out, g("to_out.0.weight"), g("to_out.0.bias"))
    rec("out", out)
    return out


def block_forward(params, x, context, temb, rotary_emb, heads, eps=1e-6, cache=None,
                  update_cache=0, candidate_rows=None, dtype=torch.float32, intermediates=None,
                  evict_order="stable"):
    """One block.  params: state_dict-named tensors; x [B, M, D]; context [B|1, Lc, D];
    temb [B, 1|M, 6, D]; rotary_emb complex64 [B|1, M, 1, hd/2] or None.
    evict_order: tie order of the KV-pool eviction (see oracle.kvcache)."""
    P = _params(params, dtype)
    eps7 = eps if isinstance(eps, (list, tuple)) else [eps] * 7
    x = x.to(dtype)
    context = context.to(dtype)
    D = x.shape[-1]
    keep = intermediates if intermediates is not None else {}
    mod = P["scale_shift_table"][None] + temb.float()
    keep["modulation"] = mod
    shift, scale, gate, c_shift, c_scale, c_gate = (mod[:, :, i] for i in range(6))
    n1 = F.layer_norm(x.float(), (D,), eps=eps7[0])
    keep["norm1"] = n1
    h = (n1 * (1.0 + scale) + shift).to(dtype)
    keep["modulated1"] = h
    a = attention(P, "attn1", h, h, rotary_emb, heads, eps7[3], eps7[4], cache, update_cache,
                  candidate_rows, evict_order, keep=keep, name="self")
    x = (x.float() + a * gate).to(dtype)
    keep["residual1"] = x
    if "norm2.weight" in P:
        n2 = F.layer_norm(x.float(), (D,), P["norm2.weight"], P["norm2.bias"], eps7[1]).to(dtype)
    else:
        n2 = x
    keep["norm2"] = n2
    a = attention(P, "attn2", n2, context, None, heads, eps7[5], eps7[6], keep=keep, name="cross")
    x = x + a
    keep["residual2"] = x
    n3 = F.layer_norm(x.float(), (D,), eps=eps7[2])
    keep["norm3"] = n3
    h = (n3 * (1.0 + c_scale) + c_shift).to(dtype)
    keep["modulated3"] = h
    f = F.linear(h, P["ffn.net.0.proj.weight"], P["ffn.net.0.proj.bias"])
    keep["ffn1"] = f
    f = F.gelu(f, approximate="tanh")
    keep["gelu"] = f
    f = F.linear(f, P["ffn.net.2.weight"], P["ffn.net.2.bias"])
    keep["ffn2"] = f
    out = (x.float() + f.float() * c_gate).to(dtype)
    keep["output"] = out
    return out
