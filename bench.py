#!/usr/bin/env python3
"""Benchmark: one Wan2.2-5B-shaped DiT block (dim 3072, 24 x 128 heads, FFN
14336, bf16) on one MI355X through the native HIP path.

Workload "L4680": B=1, 4680 video tokens (RoPE grid 6 x 26 x 30), self
attention dense over the 4680 tokens, cross attention over a 512-token text
context whose K/V are precomputed once (WholeLayerBlock.prepare_context).
A step is one block forward over that batch; inputs are resident in HBM.
Also reported: the speculative-verify layer slice "Lverify" (4 candidates x
1560 tokens over a shared 6240-token cached prefix) and a per-stage breakdown.

Prints ONE JSON line (rank 0).  Synthetic data, random-init weights.
"""
import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "wam-egale_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "DiT-block tokens/sec + µs/layer (dim3072 bf16, 1 GPU); % of MFMA peak"
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_HBM_GBS = 8000.0
STAGE_FFN1 = 12


def layer_flops(M, D, F, Lc, self_keys, batch=1):
    """Algorithmic FLOP of one block: 2MNK per GEMM + 4 * (q-k pairs) * D for
    attention; cross K/V precomputed (not counted)."""
    R = batch * M
    gemm = 2 * R * D * (3 * D + D + D + D) + 2 * 2 * R * D * F
    attn = 4 * R * self_keys * D + 4 * R * Lc * D
    return gemm, attn


def build_block(shape, dev, seed=0):
    import torch
    from wam_ops import synthetic
    from wam_ops.block import TransformerBlock
    params = synthetic.block_params(shape, seed=seed, device=dev)
    with torch.device("meta"):
        blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
    blk.load_state_dict(params, assign=True)
    return blk


class OutputMismatch(RuntimeError):
    pass


def timed_steps(fn, steps, warmup, gate=None):
    """Average ms per call of fn over `steps` calls after `warmup` calls.

    gate: a name; then the first call's output is kept and the last timed
    call's output must equal it byte for byte (the reference's timing harness
    gates every timed output the same way, 算子研究/tools/time_native.py:93-122)."""
    import torch
    first = None
    for i in range(max(warmup, 1 if gate else 0)):
        out = fn()
        if gate and i == 0:
            first = out.clone()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    last = None
    for _ in range(steps):
        last = fn()
    end.record()
    torch.cuda.synchronize()
    if gate is not None and not torch.equal(first, last):
        raise OutputMismatch(f"{gate}: the last timed output differs from the first call's")
    return start.elapsed_time(end) / steps


def graph_replay_ms(fn, steps, warmup, what):
    """Capture one call of fn into a HIP graph (torch.cuda.graph) and time
    `steps` replays; every replay's output must equal the eager output byte for
    byte.  The reference quotes its block times as warm graph replays
    (算子研究/wam_ops/optimized/prepared.py:1-4)."""
    import torch
    ref = fn().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()

    def replay():
        g.replay()
        return out
    ms = timed_steps(replay, steps, warmup, gate=what)
    if not torch.equal(out, ref):
        raise OutputMismatch(f"{what}: the graph replay's output differs from the eager call's")
    del g
    return ms


def cache_state(blocks, name="pos"):
    """Clones of every pool tensor (k, v, id, mask, is_pred) of the blocks."""
    return [{k: v.clone() for k, v in b.attn1.attn_caches[name].items()} for b in blocks]


def check_cache_state(blocks, before, what, name="pos"):
    import torch
    for i, (b, snap) in enumerate(zip(blocks, before)):
        for k, v in snap.items():
            if not torch.equal(b.attn1.attn_caches[name][k], v):
                raise OutputMismatch(f"{what}: layer {i} cache {k} changed during a read-only timed run")


def stage_times(lib, call, n_calls, mask):
    """Average ms per recorded stage over n_calls, from HIP events recorded on
    the launch stream around each selected stage."""
    from wam_ops._lib import STAGES
    timer = lib.wam_timer_create(64 * n_calls, mask)
    try:
        for _ in range(n_calls):
            call(timer)
        n = 64 * n_calls
        st = (ctypes.c_int32 * n)()
        ms = (ctypes.c_float * n)()
        got = lib.wam_timer_read(timer, st, ms, n)
        acc = {}
        for i in range(got):
            acc.setdefault(STAGES[st[i]], []).append(ms[i])
        return {k: sum(v) / len(v) for k, v in acc.items()}
    finally:
        lib.wam_timer_destroy(timer)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _time_oracle(params, x, ctx, temb, freqs, heads, eps, warmup, runs):
    import torch
    from oracle.block import block_forward
    with torch.no_grad():
        for _ in range(warmup):
            block_forward(params, x, ctx, temb, freqs, heads, eps)
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            block_forward(params, x, ctx, temb, freqs, heads, eps)
            times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], times


def cpu_baseline(l4680=True):
    """The oracle (the CPU fp32 restatement of the reference block,
    WanTransformerBlock.forward, model.py:741-794) timed on this host's cores.

    Main figure: the Wan-1.3B-shaped block (dim 1536, 12 x 128 heads, FFN 8960,
    B=1, 1024 tokens on a (4, 16, 16) grid, 512 context tokens, per-sample
    temb), fp32, 3 warmups then the median of 7 runs.  Extra: one L4680 layer
    (dim 3072, 4680 tokens) in fp32, 1 warmup then the median of 3."""
    import torch
    from wam_ops import synthetic
    threads = torch.get_num_threads()
    shape = synthetic.WAN_1_3B
    params = {k: v.float() for k, v in synthetic.block_params(shape, seed=0, device="cpu").items()}
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 1024, (4, 16, 16), context_len=512, seed=0)
    x, ctx = x.float(), ctx.float()
    med, times = _time_oracle(params, x, ctx, temb, freqs, shape.heads, shape.eps, 3, 7)
    res = {"value": round(1024 / med, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
           "ms_per_layer": round(med * 1e3, 2),
           "sample": f"C1: one Wan-1.3B-shaped block (dim 1536, 12x128 heads, FFN 8960, B=1, 1024 tokens, "
                     f"512 context tokens) in fp32 through the CPU oracle; 3 warmups, median of "
                     f"{len(times)} runs ({', '.join(f'{t * 1e3:.1f}' for t in times)} ms); torch threads "
                     f"{threads}, os.cpu_count {os.cpu_count()}, {_cpu_model()}"}
    if l4680:
        shape = synthetic.WAN22_5B
        params = {k: v.float() for k, v in synthetic.block_params(shape, seed=0, device="cpu").items()}
        x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 4680, (6, 26, 30), context_len=512, seed=1)
        med, times = _time_oracle(params, x.float(), ctx.float(), temb, freqs, shape.heads, shape.eps, 1, 3)
        res["l4680"] = {"tokens_per_s": round(4680 / med, 1), "ms_per_layer": round(med * 1e3, 1),
                        "sample": "one L4680 layer (B=1, 4680 tokens, dim 3072, fp32) through the CPU oracle, "
                                  f"1 warmup, median of {len(times)}"}
    return res


def mfma_peaks(lib, dev, iters=20000, reps=3):
    """Measured dense MFMA throughput (TFLOP/s) of the probe kernel, best of
    `reps` launches, for bf16 and fp8 e4m3 in both MFMA shapes."""
    import torch
    from wam_ops import _lib
    from wam_ops.ops import stream_handle
    sink = torch.empty(2 * torch.cuda.get_device_properties(dev).multi_processor_count * 256,
                       dtype=torch.float32, device=dev)
    out = {}
    for name, kind in (("bf16_32x32x16", _lib.PEAK_BF16_32), ("bf16_16x16x32", _lib.PEAK_BF16_16),
                       ("fp8_32x32x64", _lib.PEAK_FP8_32), ("fp8_16x16x128", _lib.PEAK_FP8_16)):
        flop = ctypes.c_double()
        best = 0.0
        for _ in range(reps + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            _lib.check(lib.wam_mfma_peak(kind, iters, ctypes.c_void_p(sink.data_ptr()), sink.numel() * 4,
                                         ctypes.byref(flop), stream_handle(dev)), "wam_mfma_peak")
            b.record()
            torch.cuda.synchronize()
            best = max(best, flop.value / (a.elapsed_time(b) * 1e-3) / 1e12)
        out[name] = round(best, 1)
    return out


TRAFFIC_FILE = ROOT / "profiles" / "l4680_ffn1_traffic.md"


def pmc_ffn1(shape, dev, M):
    """Counter-pass workload: the L4680 FFN1 GEMM (LN3 output [M, 3072] x
    W1 [14336, 3072]^T + b1, GELU) 5 times, then a plain 1 GiB device-to-device
    copy 3 times, whose FETCH_SIZE / WRITE_SIZE calibrate the counters."""
    import torch
    from wam_ops import ops
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(M, shape.dim, device=dev, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(shape.ffn, shape.dim, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    b1 = torch.zeros(shape.ffn, device=dev, dtype=torch.bfloat16)
    for _ in range(5):
        ops.linear(x, w1, b1, epilogue=ops.EPI_BIAS_GELU)
    torch.cuda.synchronize()
    src = torch.ones(1 << 29, device=dev, dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_ffn1": "done", "copy_bytes": src.numel() * 2}), flush=True)


def pmc_attn(shape, dev, M):
    """Counter-pass workload for the attention kernels, 5 launches each, in
    this order: self-attention over the packed QKV of the L4680 block (M
    queries and M keys, 24 heads of 128), cross-attention of the same queries
    over 512 text keys, and the C4a unit (1560 queries over 6240 cached pool
    keys read through a slot list plus 1560 own keys)."""
    import torch
    from wam_ops import ops
    g = torch.Generator(device=dev).manual_seed(11)
    H, hd = shape.heads, shape.dim // shape.heads
    r = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)
    qkv = r(1, M, 3, H, hd)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    kc, vc = r(1, 512, H, hd), r(1, 512, H, hd)
    q1, k1, v1 = r(1, 1560, H, hd), r(1, 1560, H, hd), r(1, 1560, H, hd)
    pk, pv = r(1, 6240, H, hd), r(1, 6240, H, hd)
    slots = torch.arange(6240, dtype=torch.int32, device=dev)
    n_hist = torch.tensor([6240], dtype=torch.int32, device=dev)
    for _ in range(5):
        ops.attention(q, k, v)
    for _ in range(5):
        ops.attention(q, kc, vc)
    for _ in range(5):
        ops.attention(q1, k1, v1, pool_k=pk, pool_v=pv, slots=slots, n_hist=n_hist)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_attn": "done"}), flush=True)


def measured_traffic():
    """HBM bytes per FFN1 launch from the committed counter summary (two
    rocprofv3 --pmc passes, each calibrated against a 1 GiB copy), or None."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def _unit(ms, flop):
    return {"us": round(ms * 1e3, 1), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
            "frac_of_bf16_peak": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}


def c4a_attention(shape, dev, steps, warmup, q_tokens=1560, prefix=6240):
    """Self attention of 1560 new tokens over a 6240-token cached prefix (pool
    row 0, slots 0..6239) plus themselves, 24 x 128 heads; N(0, 1) Q/K/V.  The
    history base is passed as the block passes kv_layout's info[2] (the
    prefix is one run of consecutive slots)."""
    import torch
    from wam_ops import ops
    H = shape.heads
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn(1, q_tokens, H, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(1, q_tokens, H, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(1, q_tokens, H, 128, generator=g, device=dev).to(torch.bfloat16)
    pk = torch.randn(1, prefix, H, 128, generator=g, device=dev).to(torch.bfloat16)
    pv = torch.randn(1, prefix, H, 128, generator=g, device=dev).to(torch.bfloat16)
    slots = torch.arange(prefix, dtype=torch.int32, device=dev)
    n_hist = torch.tensor([prefix], dtype=torch.int32, device=dev)
    base = torch.zeros(1, dtype=torch.int32, device=dev)
    ms = timed_steps(lambda: ops.attention(q, k, v, pool_k=pk, pool_v=pv, slots=slots, n_hist=n_hist,
                                           hist_base=base),
                     steps, warmup, gate="C4a self attention")
    return _unit(ms, 4 * q_tokens * (prefix + q_tokens) * shape.dim)


def verify_stack30(shape, dev, x, ctx, temb, freqs, rows, prefix, steps, warmup, layers=30):
    """C5: the 30-layer speculative verify forward, measured two ways over the
    same 30 random-init layers (each with its own 6240-token committed prefix
    in pool row 0); 4 candidates x 1560 tokens:

    stack30 - the block loop alone (BlockStack, precomputed cross K/V);
    model30 - the whole WanTransformer3DModel forward (WholeModel): patch
              embedding of [4, 48, 2, 52, 60] latents, RoPE from grid ids, the
              condition embedder on the [4, 2] per-frame timesteps, the 30
              blocks, norm_out + modulation and proj_out, with the 512 x 4096
              text prepared once (text embedder + every layer's cross K/V)."""
    import torch
    from wam_ops import BlockStack, TransformerModel, synthetic
    B, Mv = x.shape[0], x.shape[1]
    blocks = []
    for i in range(layers):
        blk = build_block(shape, dev, seed=100 + i)
        blk.attn1.attn_caches["pos"] = synthetic.kv_pool(shape, prefix + Mv, prefix, batch=1,
                                                         seed=300 + i, device=dev)
        blocks.append(blk)
    stack = BlockStack(blocks)
    with torch.no_grad():
        stack.prepare_context(ctx, precompute=True)

    def run():
        with torch.no_grad():
            return stack(x, ctx, temb, freqs, candidate_cache_rows=rows)
    before = cache_state(blocks)
    ms = timed_steps(run, steps, warmup, gate="stack30")
    check_cache_state(blocks, before, "stack30")
    g, a = layer_flops(Mv, shape.dim, shape.ffn, ctx.shape[1], self_keys=prefix + Mv, batch=B)
    res = {"layers": layers, "ms_per_forward": round(ms, 3), "us_per_layer": round(ms * 1e3 / layers, 1),
           "tokens_per_s": round(B * Mv / (ms * 1e-3), 1),
           "tflops": round(layers * (g + a) / (ms * 1e-3) / 1e12, 1), "steps": steps, "warmup": warmup}
    del stack

    # the whole model over the same layers
    with torch.device("meta"):
        model = TransformerModel(num_attention_heads=shape.heads, attention_head_dim=shape.head_dim,
                                 ffn_dim=shape.ffn, num_layers=0)
    model.load_state_dict(synthetic.model_io_params(model, seed=7, device=dev), assign=True)
    model.blocks = torch.nn.ModuleList(blocks)
    gen = torch.Generator(device=dev).manual_seed(11)
    frames, hp, wp = 2, 26, 30
    lat = torch.randn(B, 48, frames, 2 * hp, 2 * wp, generator=gen, device=dev).to(torch.bfloat16)
    text = torch.randn(1, ctx.shape[1], 4096, generator=gen, device=dev).to(torch.bfloat16)
    grid = synthetic.mesh_grid_ids(frames, hp, wp).to(torch.int64)
    grid = torch.cat([grid, torch.zeros_like(grid[:1])])[None].repeat(B, 1, 1).to(dev)
    inp = {"noisy_latents": lat, "text_emb": text.expand(B, -1, -1).clone(), "grid_id": grid,
           "timesteps": torch.tensor([[0.0, 500.0 + 50 * k] for k in range(B)], device=dev)}
    whole = model.native()
    with torch.no_grad():
        prep_ms = timed_steps(lambda: whole.prepare_text(inp["text_emb"]), 1, 1)

        def model_step():
            return whole(inp, candidate_cache_rows=rows)

        def io_step():
            xe = whole.embed(lat, False)
            fr = whole._bind()
            from wam_ops import ops
            ops.rope_freqs(grid)
            te, _ = fr["cond"].time(inp["timesteps"], xe.dtype)
            return whole.head(xe, te, False)
        mms = timed_steps(model_step, steps, warmup, gate="model30")
        ims = timed_steps(io_step, steps, warmup, gate="model30 I/O")
    check_cache_state(blocks, before, "model30")
    res_model = {"ms_per_forward": round(mms, 3), "tokens_per_s": round(B * Mv / (mms * 1e-3), 1),
                 "io_us": round(ims * 1e3, 1), "prepare_text_ms": round(prep_ms, 3),
                 "latents": list(lat.shape), "text": [B, ctx.shape[1], 4096], "timesteps": [B, frames]}
    del whole, model, blocks
    torch.cuda.empty_cache()
    return res, res_model


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--pmc-ffn1", action="store_true",
                    help="only launch the FFN1 GEMM 5 times and a 1 GiB device copy 3 times "
                         "(the workload for the FETCH_SIZE / WRITE_SIZE counter passes)")
    ap.add_argument("--pmc-attn", action="store_true",
                    help="only launch self-, cross- and C4a attention 5 times each "
                         "(the workload for the attention instruction-count passes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the block runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured path).", file=sys.stderr)
        sys.exit(2)

    import torch
    from wam_ops import _lib, synthetic
    from wam_ops.whole_layer import WholeLayerBlock
    lib = _lib.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    shape = synthetic.WAN22_5B
    D, F, M, Lc = shape.dim, shape.ffn, 4680, 512

    if args.pmc_ffn1:
        pmc_ffn1(shape, dev, M)
        return
    if args.pmc_attn:
        pmc_attn(shape, dev, M)
        return

    blk = build_block(shape, dev)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, M, (6, 26, 30), context_len=Lc,
                                                 seed=1, device=dev)
    layer = WholeLayerBlock(blk)
    with torch.no_grad():
        layer.prepare_context(ctx, precompute=True)
    torch.cuda.synchronize()

    def step(timer=None):
        with torch.no_grad():
            return layer(x, ctx, temb, freqs, timer=timer)

    ms = timed_steps(step, args.steps, args.warmup, gate="L4680")
    gms = graph_replay_ms(step, args.steps, args.warmup, "L4680 graph replay")
    # Dominant kernel (FFN1 GEMM + GELU): HIP events around its launch on the
    # launch stream, over the same number of steps.
    ffn1 = stage_times(lib, step, args.steps, 1 << STAGE_FFN1)["ffn1"]
    stages = stage_times(lib, step, 3, (1 << len(_lib.STAGES)) - 1)

    peaks = mfma_peaks(lib, dev)
    peak_meas = peaks["bf16_32x32x16"]
    gemm, attn = layer_flops(M, D, F, Lc, self_keys=M)
    flops = gemm + attn
    ffn1_flops = 2 * M * D * F
    ffn1_tflops = ffn1_flops / (ffn1 * 1e-3) / 1e12
    layer_tflops = flops / (ms * 1e-3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(M / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "us_per_layer": round(ms * 1e3, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1) activations, N(0,0.02) random-init weights)",
        "config": {"workload": "L4680: one Wan2.2-5B DiT block, B=1, 4680 tokens (RoPE grid 6x26x30), "
                               "dim 3072, 24x128 heads, FFN 14336, dense self-attention over 4680, "
                               "cross-attention over 512 precomputed text K/V",
                   "tokens": M, "dim": D, "heads": shape.heads, "ffn": F, "context": Lc},
        "layer_tflops": round(layer_tflops, 1),
        "layer_frac_of_bf16_peak": round(layer_tflops / PEAK_BF16_TFLOPS, 4),
        "layer_frac_of_measured_bf16_peak": round(layer_tflops / peak_meas, 4),
        "layer_flop": flops,
        "roofline": {"bound": "mfma", "kernel": "FFN1 GEMM 4680x14336x3072 + bias + GELU(tanh)",
                     "achieved": round(ffn1_tflops, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ffn1_tflops / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(),
                     "traffic_source": ("profiles/" + TRAFFIC_FILE.name + " (rocprofv3 FETCH_SIZE and "
                                        "WRITE_SIZE passes over bench.py --pmc-ffn1; not measured in "
                                        "this run)"),
                     "kernel_us": round(ffn1 * 1e3, 1),
                     "peak_measured": peak_meas,
                     "frac_of_measured": round(ffn1_tflops / peak_meas, 4)},
        "mfma_peak_tflops": {"vendor": {"bf16": PEAK_BF16_TFLOPS, "fp8": PEAK_FP8_TFLOPS},
                             "measured": peaks},
        "outputs_checked": "every timed loop's last output equals its first call's byte for byte; "
                           "read-only KV pools unchanged",
        "stages_us": {k: round(v * 1e3, 1) for k, v in stages.items()},
        "graph_replay": {"us_per_layer": round(gms * 1e3, 1), "tokens_per_s": round(M / (gms * 1e-3), 1),
                         "checked": "the layer captured once into a HIP graph; every timed replay's "
                                    "output equals the eager call's byte for byte"},
    }
    # Per-unit lines of the same run (algorithmic FLOP as in the layer count):
    # C2 QKV + q/k RMSNorm + RoPE, C3 FFN (FFN1 + GELU + FFN2 + gated
    # residual), C4b cross attention over 512 keys, from the stage timers of
    # the layer; C4a self attention (1560 queries over a 6240-token cached
    # prefix + themselves) as its own call.
    out["units"] = {
        "C2_qkv_rms_rope": _unit(stages["qkv"] + stages["rms_rope"], 2 * M * D * 3 * D),
        "C3_ffn": _unit(stages["ffn1"] + stages["ffn2"], 2 * 2 * M * D * F),
        "C4b_cross_attention": _unit(stages["cross_attn"], 4 * M * Lc * D),
        "C4a_self_attention": c4a_attention(shape, dev, args.steps, args.warmup),
    }
    # C3 variants: the same layer with e4m3 FFN weights (per-output-channel
    # fp32 scales) and bf16 activations, and with FFN1's input quantized too
    # (per-row scales, inside LayerNorm 3; FFN1 on the fp8 MFMA); everything
    # else unchanged.
    ffn_flops = 2 * 2 * M * D * F
    variants = {
        "fp8_ffn_variant": (dict(ffn_fp8=True),
                            "e4m3 per-output-channel scales (absmax/448), bf16 activations, fp32 accumulate"),
        "fp8_act_ffn_variant": (dict(ffn_fp8=True, ffn_act_fp8=1),
                                "e4m3 weights as above; FFN1 input e4m3 with per-row scales (absmax/448, "
                                "written by LayerNorm 3) on the fp8 MFMA; FFN2 bf16 activations"),
        "fp8_mx_ffn_variant": (dict(ffn_fp8=True, ffn_act_fp8=2),
                               "e4m3 weights as above; FFN1 input e4m3 with per-row scales on the fp8 MFMA; "
                               "hidden layer e4m3 with one e8m0 exponent per 32 values (MX), FFN2 on the fp8 "
                               "MFMA with those block scales"),
    }
    for key, (opts, what) in variants.items():
        flayer = WholeLayerBlock(blk, **opts)
        with torch.no_grad():
            flayer.prepare_context(ctx, precompute=True)

        def fstep(timer=None):
            with torch.no_grad():
                return flayer(x, ctx, temb, freqs, timer=timer)
        fms = timed_steps(fstep, args.steps, args.warmup, gate=f"L4680 {key}")
        fst = stage_times(lib, fstep, 3, (1 << len(_lib.STAGES)) - 1)
        out[key] = {
            "us_per_layer": round(fms * 1e3, 1), "tokens_per_s": round(M / (fms * 1e-3), 1),
            "ffn_unit_us": round((fst["ffn1"] + fst["ffn2"]) * 1e3, 1),
            "ffn1_us": round(fst["ffn1"] * 1e3, 1), "ln3_us": round(fst["ln3"] * 1e3, 1),
            "ffn_unit_us_bf16": round((stages["ffn1"] + stages["ffn2"]) * 1e3, 1),
            "ffn_unit_tflops": round(ffn_flops / ((fst["ffn1"] + fst["ffn2"]) * 1e-3) / 1e12, 1),
            "weights": what,
        }
        del flayer
    if not args.no_verify:
        # Lverify: 4 candidates x 1560 tokens, each over the shared 6240-token
        # prefix (pool row 0) plus its own 1560 tokens; read-only cache.
        Mv, B, prefix = 1560, 4, 6240
        xv, ctxv, tembv, freqv = synthetic.block_inputs(shape, B, Mv, (2, 26, 30), context_len=Lc,
                                                        seed=2, device=dev)
        blk.attn1.attn_caches["pos"] = synthetic.kv_pool(shape, prefix + Mv, prefix, batch=1, device=dev)
        rows = torch.zeros(B, dtype=torch.int64, device=dev)
        vlayer = WholeLayerBlock(blk)
        with torch.no_grad():
            vlayer.prepare_context(ctxv, precompute=True)

        def vstep():
            with torch.no_grad():
                return vlayer(xv, ctxv, tembv, freqv, candidate_cache_rows=rows)
        # candidate_cache_rows are read back and validated on the host the first time this
        # tensor is seen (again after any in-place write), as the reference checks them
        vbefore = cache_state([blk])
        vms = timed_steps(vstep, args.steps, args.warmup, gate="Lverify")
        check_cache_state([blk], vbefore, "Lverify")
        g, a = layer_flops(Mv, D, F, Lc, self_keys=prefix + Mv, batch=B)
        out["lverify"] = {"tokens": B * Mv, "us_per_layer": round(vms * 1e3, 1),
                          "tokens_per_s": round(B * Mv / (vms * 1e-3), 1),
                          "tflops": round((g + a) / (vms * 1e-3) / 1e12, 1),
                          "frac_of_bf16_peak": round((g + a) / (vms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                          "us_30_layers_extrapolated": round(30 * vms * 1e3, 1)}
        del vlayer
        out["lverify"]["stack30"], out["lverify"]["model30"] = verify_stack30(
            shape, dev, xv, ctxv, tembv, freqv, rows, prefix, min(args.steps, 5), 2)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
