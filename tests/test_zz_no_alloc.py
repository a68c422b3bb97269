"""ab_ibcs_sip_static (libab_attention_static.so), the fused plan without
allocation (its IBCS intermediates live in a static device array of
AB_STATIC_SCRATCH_BYTES per GPU, in that library's code object), against
ab_ibcs_sip with a caller workspace: ids and weights must be
the same bits. Two calls in a row, the second smaller, so the second runs
over what the first left in the shared array: 3 heads of the Wan2.1-14B
720p length (two head chunks of the 512 MiB array), then 2 heads of 8,192
tokens read through a token order. A head too long for the array is
rejected before any launch. The whole call, the static plan then the prefill,
recorded into one HIP graph replays with new inputs to the eager bits. The
first test, run before anything else loads the static library in this
process, reports the device memory the array takes and when."""
import pytest
import torch

from ab_attention import _lib

pytestmark = pytest.mark.gpu


def _inputs(heads, n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(1, heads, n, 128, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(1, heads, n, 128, device="cuda", generator=g).to(torch.bfloat16)
    rows = heads * -(-n // 128)
    offsets = torch.rand(rows, device="cuda", generator=g)
    return q, k, offsets


def _with_workspace(lib, q, k, order, offsets, samples):
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    rows = offsets.shape[0]
    ids = torch.empty(rows, samples, dtype=torch.int32, device="cuda")
    w = torch.empty(rows, samples, dtype=torch.float32, device="cuda")
    ws_bytes = lib.ab_ibcs_sip_workspace_bytes(bh, n)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    _lib.check(lib.ab_ibcs_sip(_lib.ptr(q), _lib.ptr(k), _lib.ptr(order), bh, n, _lib.ptr(offsets), samples,
                               _lib.ptr(ws), ws_bytes, _lib.ptr(ids), _lib.ptr(w), _lib.stream(q.device)))
    return ids, w


def _free_bytes():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return torch.cuda.mem_get_info()[0]


def test_static_scratch_reserved_by_static_library_only():
    """The main library has no static array: only loading (or first calling)
    libab_attention_static.so takes AB_STATIC_SCRATCH_BYTES of device memory."""
    if _lib._static is not None:
        pytest.skip("the static library was already loaded in this process")
    lib = _lib.load()
    heads, n, samples = 1, 8192, 256
    q, k, offsets = _inputs(heads, n, 7)
    ids_r, w_r = _with_workspace(lib, q, k, None, offsets, samples)  # main library code object in use
    del ids_r, w_r
    ids = torch.empty(offsets.shape[0], samples, dtype=torch.int32, device="cuda")
    w = torch.empty(offsets.shape[0], samples, dtype=torch.float32, device="cuda")
    before = _free_bytes()
    static = _lib.load_static()
    after_load = _free_bytes()
    _lib.check(static.ab_ibcs_sip_static(_lib.ptr(q), _lib.ptr(k), None, heads, n, _lib.ptr(offsets), samples,
                                         _lib.ptr(ids), _lib.ptr(w), _lib.stream(q.device)))
    after_call = _free_bytes()
    mib = 1 << 20
    print(f"static scratch: device memory taken by loading the library {(before - after_load) / mib:.1f} MiB, "
          f"by its first call {(after_load - after_call) / mib:.1f} MiB", flush=True)
    assert before - after_call >= 512 * mib  # the array is on the device once the entry point has run


def _static(lib, q, k, order, offsets, samples):
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    rows = offsets.shape[0]
    ids = torch.full((rows, samples), -7, dtype=torch.int32, device="cuda")
    w = torch.full((rows, samples), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _lib.check(_lib.load_static().ab_ibcs_sip_static(_lib.ptr(q), _lib.ptr(k), _lib.ptr(order), bh, n,
                                                     _lib.ptr(offsets), samples, _lib.ptr(ids), _lib.ptr(w),
                                                     _lib.stream(q.device)))
    return ids, w


def test_static_plan_equals_workspace_plan():
    lib = _lib.load()
    for heads, n, samples, ordered, seed in ((3, 75600, 2048, False, 1), (2, 8192, 256, True, 2)):
        print(f"static plan heads={heads} n={n} samples={samples} ordered={ordered}", flush=True)
        q, k, offsets = _inputs(heads, n, seed)
        order = (torch.randperm(n, generator=torch.Generator().manual_seed(seed)).to(torch.int32).cuda()
                 if ordered else None)
        ids_s, w_s = _static(lib, q, k, order, offsets, samples)
        torch.cuda.synchronize()
        ids_r, w_r = _with_workspace(lib, q, k, order, offsets, samples)
        torch.cuda.synchronize()
        assert torch.equal(ids_s, ids_r)
        assert torch.equal(w_s.view(torch.int32), w_r.view(torch.int32))


def test_static_plan_rejects_oversized_head():
    lib = _lib.load()
    n = 131072
    q = torch.zeros(1, 1, 4096, 128, dtype=torch.bfloat16, device="cuda")  # never read: rejected first
    rc = _lib.load_static().ab_ibcs_sip_static(_lib.ptr(q), _lib.ptr(q), None, 1, n, _lib.ptr(q), 2048,
                                               _lib.ptr(q), _lib.ptr(q), _lib.stream(q.device))
    assert rc == 1
    assert b"static scratch" in lib.ab_last_error()


def test_static_plan_in_hip_graph():
    """The case the entry point is for: the plan (ab_ibcs_sip_static) and the
    prefill over it recorded into one HIP graph, with every buffer allocated
    before capture. Each replay, after new Q/K/V and uniforms are copied into
    the captured inputs (with eager work and synchronisations between
    replays), equals ab_ibcs_sip with a workspace plus the prefill, bit for
    bit."""
    lib = _lib.load()
    static = _lib.load_static()
    heads, n, samples = 2, 8192, 256
    q, k, offsets = _inputs(heads, n, 3)
    v = torch.randn(1, heads, n, 128, device="cuda").to(torch.bfloat16)
    rows = offsets.shape[0]
    ids = torch.empty(rows, samples, dtype=torch.int32, device="cuda")
    w = torch.empty(rows, samples, dtype=torch.float32, device="cuda")
    out = torch.empty_like(q)
    lse = torch.empty(1, heads, n, dtype=torch.float32, device="cuda")

    def call(stream):
        _lib.check(static.ab_ibcs_sip_static(_lib.ptr(q), _lib.ptr(k), None, heads, n, _lib.ptr(offsets),
                                             samples, _lib.ptr(ids), _lib.ptr(w), stream))
        _lib.check(lib.ab_paged_prefill(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), heads, n, _lib.ptr(ids),
                                        _lib.ptr(w), samples, _lib.ptr(out), _lib.ptr(lse), stream))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(_lib.stream(q.device))  # first call on the device outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(_lib.stream(q.device))
    for i in range(3):
        print(f"static plan graph replay {i}", flush=True)
        g = torch.Generator(device="cuda").manual_seed(40 + i)
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, device="cuda", generator=g).to(torch.bfloat16))
        offsets.copy_(torch.rand(rows, device="cuda", generator=g))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (ids.clone(), w.clone(), out.clone(), lse.clone())
        ids_r, w_r = _with_workspace(lib, q, k, None, offsets, samples)
        out_r, lse_r = torch.empty_like(q), torch.empty_like(lse)
        _lib.check(lib.ab_paged_prefill(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), heads, n, _lib.ptr(ids_r),
                                        _lib.ptr(w_r), samples, _lib.ptr(out_r), _lib.ptr(lse_r),
                                        _lib.stream(q.device)))
        torch.cuda.synchronize()
        assert torch.equal(got[0], ids_r) and torch.equal(got[1].view(torch.int32), w_r.view(torch.int32))
        assert torch.equal(got[2].view(torch.int16), out_r.view(torch.int16)) and torch.equal(got[3], lse_r)
