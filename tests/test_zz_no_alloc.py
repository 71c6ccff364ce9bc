"""wam_attention_noalloc: wam_attention without a workspace or any device
allocation (the key-range split's partials in the library's static scratch).

Called through the C ABI and compared with wam_attention given a workspace of
wam_attention_workspace_bytes (the same split plan): the outputs must be
bitwise equal, on two calls in a row, the second with a smaller input, both
of which run a key-range split.  A shape whose split needs more than the
64 MiB scratch, and a call that passes a workspace, are refused on the host.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

H = 24
MIB = 1 << 20


def _inputs(dev, B, Mq, prefix, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)
    q, k, v = r(B, Mq, H, 128), r(B, Mq, H, 128), r(B, Mq, H, 128)
    pk, pv = r(1, prefix, H, 128), r(1, prefix, H, 128)
    slots = torch.arange(prefix, dtype=torch.int32, device=dev)
    n_hist = torch.tensor([prefix], dtype=torch.int32, device=dev)
    rows = torch.zeros(B, dtype=torch.int64, device=dev)
    return q, k, v, pk, pv, slots, n_hist, rows


def _args(q, k, v, pk, pv, slots, n_hist, rows, o, max_keys=None):
    from wam_ops import _lib
    a = _lib.AttentionArgs()
    B, Mq, Hh, hd = q.shape
    a.q, a.q_bstride, a.q_rstride = q.data_ptr(), q.stride(0), q.stride(1)
    a.o, a.o_bstride, a.o_rstride = o.data_ptr(), o.stride(0), o.stride(1)
    a.B, a.Mq, a.H, a.head_dim = B, Mq, Hh, hd
    a.pool_k, a.pool_v = pk.data_ptr(), pv.data_ptr()
    a.pool_bstride, a.pool_rstride, a.pool_batch = pk.stride(0), pk.stride(1), pk.shape[0]
    a.slots, a.n_hist_dev, a.pool_rows = slots.data_ptr(), n_hist.data_ptr(), rows.data_ptr()
    a.k, a.v, a.kv_bstride, a.kv_rstride = k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1)
    a.Mk, a.kv_batch = k.shape[1], k.shape[0]
    a.scale = 1.0 / 128 ** 0.5
    a.max_keys = max_keys if max_keys is not None else k.shape[1] + pk.shape[1]
    return a


def _err():
    from wam_ops import _lib
    return _lib.lib().wam_last_error().decode()


def test_noalloc_matches_workspace_entry_point(dev):
    from wam_ops import _lib
    from wam_ops.ops import stream_handle
    lib = _lib.lib()
    s = stream_handle(dev)
    # the verify layer's self attention (4 x 1560 queries over 6240 cached +
    # 1560 own keys), then a smaller call; both plans split the last round
    for B, Mq, prefix, seed in ((4, 1560, 6240, 1), (1, 520, 2000, 2)):
        print(f"noalloc attention B={B} Mq={Mq} prefix={prefix}", flush=True)
        x = _inputs(dev, B, Mq, prefix, seed)
        o_ref = torch.empty_like(x[0])
        o_got = torch.full_like(x[0], float("nan"))
        a = _args(*x, o_ref)
        need = lib.wam_attention_workspace_bytes(a.B, a.Mq, a.H, a.max_keys)
        assert 0 < need <= 64 * MIB, need
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
        assert lib.wam_attention(ctypes.byref(a), s) == _lib.WAM_OK, _err()
        b = _args(*x, o_got)
        assert lib.wam_attention_noalloc(ctypes.byref(b), s) == _lib.WAM_OK, _err()
        torch.cuda.synchronize()
        assert torch.equal(o_got, o_ref), f"B={B} Mq={Mq}: no-alloc output differs"


def _args_own(q, k, v, o):
    """Own keys only (no pool): the pipelined kernel's 224-query units."""
    from wam_ops import _lib
    a = _lib.AttentionArgs()
    B, Mq, Hh, hd = q.shape
    a.q, a.q_bstride, a.q_rstride = q.data_ptr(), q.stride(0), q.stride(1)
    a.o, a.o_bstride, a.o_rstride = o.data_ptr(), o.stride(0), o.stride(1)
    a.B, a.Mq, a.H, a.head_dim = B, Mq, Hh, hd
    a.k, a.v, a.kv_bstride, a.kv_rstride = k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1)
    a.Mk, a.kv_batch = k.shape[1], k.shape[0]
    a.scale = 1.0 / 128 ** 0.5
    a.max_keys = k.shape[1]
    return a


def test_noalloc_own_keys_split_matches(dev):
    from wam_ops import _lib
    from wam_ops.ops import stream_handle
    lib = _lib.lib()
    s = stream_handle(dev)
    # 1560 queries over 7800 own keys, then 1300 over 3000: both plans run
    # 224-query units in 3 key ranges (59 MB, then 50 MB of partial results)
    for Mq, Mk, seed in ((1560, 7800, 5), (1300, 3000, 6)):
        print(f"noalloc own-key attention Mq={Mq} Mk={Mk}", flush=True)
        g = torch.Generator(device=dev).manual_seed(seed)
        r = lambda *sh: torch.randn(*sh, generator=g, device=dev).to(torch.bfloat16)
        q, k, v = r(1, Mq, H, 128), r(1, Mk, H, 128), r(1, Mk, H, 128)
        o_ref = torch.empty_like(q)
        o_got = torch.full_like(q, float("nan"))
        a = _args_own(q, k, v, o_ref)
        need = lib.wam_attention_workspace_bytes(a.B, a.Mq, a.H, a.max_keys)
        assert 0 < need <= 64 * MIB, need
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
        assert lib.wam_attention(ctypes.byref(a), s) == _lib.WAM_OK, _err()
        b = _args_own(q, k, v, o_got)
        assert lib.wam_attention_noalloc(ctypes.byref(b), s) == _lib.WAM_OK, _err()
        torch.cuda.synchronize()
        assert torch.equal(o_got, o_ref), f"Mq={Mq} Mk={Mk}: no-alloc output differs"


def test_noalloc_refuses_on_host(dev):
    from wam_ops import _lib
    from wam_ops.ops import stream_handle
    lib = _lib.lib()
    s = stream_handle(dev)
    x = _inputs(dev, 4, 200, 200, 3)
    o = torch.empty_like(x[0])
    # a key bound of 16000 makes the split plan need 97.5 MiB of partials
    a = _args(*x, o, max_keys=16000)
    assert lib.wam_attention_workspace_bytes(a.B, a.Mq, a.H, a.max_keys) > 64 * MIB
    assert lib.wam_attention_noalloc(ctypes.byref(a), s) == _lib.WAM_ERR_ARG
    assert "maximum" in _err()
    a = _args(*x, o)
    ws = torch.empty(1024, dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), 1024
    assert lib.wam_attention_noalloc(ctypes.byref(a), s) == _lib.WAM_ERR_ARG
    assert "no workspace" in _err()


def test_noalloc_under_graph_capture(dev):
    """What the entry point is for: after one warm-up call (which looks the
    scratch address up), a call captured into a HIP graph allocates nothing,
    and every replay equals the eager output bit for bit, with the program's
    own eager work and synchronisations between the replays."""
    from wam_ops import _lib
    from wam_ops.ops import stream_handle
    lib = _lib.lib()
    x = _inputs(dev, 4, 1560, 6240, 7)  # a split plan (160 units in 3 key ranges)
    o_eager = torch.empty_like(x[0])
    a = _args(*x, o_eager)
    assert lib.wam_attention_workspace_bytes(a.B, a.Mq, a.H, a.max_keys) > 0
    assert lib.wam_attention_noalloc(ctypes.byref(a), stream_handle(dev)) == _lib.WAM_OK, _err()
    torch.cuda.synchronize()
    o_graph = torch.full_like(x[0], float("nan"))
    b = _args(*x, o_graph)
    # torch's own one-time capture state (its generator bookkeeping) comes
    # with the first capture of the process: capture a torch op once first
    warm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(warm):
        o_graph.mul_(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    before = torch.cuda.memory_allocated(dev)
    with torch.cuda.graph(graph):
        rc = lib.wam_attention_noalloc(ctypes.byref(b), stream_handle(dev))
    assert rc == _lib.WAM_OK, _err()
    grown = torch.cuda.memory_allocated(dev) - before
    assert grown == 0, f"the captured call allocated {grown} bytes of device memory"
    for i in range(3):
        print(f"noalloc graph replay {i}", flush=True)
        o_graph.fill_(float("nan"))
        x[0].add_(0)  # eager work on the inputs between replays (values unchanged)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_graph, o_eager), f"replay {i} differs from the eager call"
