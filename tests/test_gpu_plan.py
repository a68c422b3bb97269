"""The fused plan (_C.ibcs_sip / ab_ibcs_sip, used by build_plan) against the
reference-structured path (_C.ibcs then _C.sip, csrc/bindings.cpp:3-8):
SIP ids and weights must be bit-identical, since the fused kernel computes
each row's masses with the masses kernel's arithmetic straight into LDS."""
import pytest
import torch

from ab_attention import _C, _lib, build_plan
from ab_attention.synthetic import CONFIGS, make_qkv

pytestmark = pytest.mark.gpu


def _both(q, k, samples, order=None, seed=0):
    b, h, n, _ = q.shape
    rows = b * h * -(-n // 128)
    offsets = torch.rand(rows, generator=torch.Generator().manual_seed(seed)).cuda()
    ids_f = torch.empty(rows, samples, dtype=torch.int32, device="cuda")
    w_f = torch.empty(rows, samples, dtype=torch.float32, device="cuda")
    _C.ibcs_sip(q, k, offsets, ids_f, w_f, order)
    scores = _C.ibcs(q, k) if order is None else _C.ibcs_ordered(q, k, order)
    ids_s = torch.empty_like(ids_f)
    w_s = torch.empty_like(w_f)
    _C.sip(scores, offsets, ids_s, w_s)
    torch.cuda.synchronize()
    return ids_f, w_f, ids_s, w_s


def _assert_same(ids_f, w_f, ids_s, w_s):
    assert torch.equal(ids_f, ids_s)
    assert torch.equal(w_f.view(torch.int32), w_s.view(torch.int32))


@pytest.mark.parametrize("n,heads,samples", [(2048, 2, 64), (32760, 1, 2048), (1000, 3, 32)])
def test_fused_plan_equals_ibcs_then_sip(n, heads, samples):
    """c0, one full-length c1 head (8,190 blocks: a ragged last group of 8), a
    ragged query block."""
    print(f"fused plan n={n} heads={heads} samples={samples}", flush=True)
    cfg = CONFIGS[1] if n == 32760 else CONFIGS[0]
    if n == 32760:
        q, k, _ = make_qkv(cfg, heads=[0], dtype=torch.bfloat16)
        q, k = q[:1], k[:1]
    else:
        torch.manual_seed(n + heads)
        q, k = (torch.randn(1, heads, n, 128).to(torch.bfloat16) for _ in range(2))
    _assert_same(*_both(q.cuda().contiguous(), k.cuda().contiguous(), samples))


def test_fused_plan_ordered():
    """Tokens read through a permutation (the cube layout's path)."""
    print("fused plan ordered n=4096", flush=True)
    torch.manual_seed(3)
    n = 4096
    q, k = (torch.randn(1, 2, n, 128).to(torch.bfloat16).cuda() for _ in range(2))
    order = torch.randperm(n, generator=torch.Generator().manual_seed(5)).to(torch.int32).cuda()
    _assert_same(*_both(q, k, 256, order=order, seed=1))


@pytest.mark.parametrize("n", [108000, 131072])
def test_fused_plan_large_rows(n):
    """27,000 and 32,768 (the most the API accepts) blocks per row: the full
    fp64 prefix array does not fit in LDS beside the masses, so the fused kernel
    keeps 16 and 8 prefixes per chunk."""
    print(f"fused plan large rows n={n}", flush=True)
    torch.manual_seed(8)
    q, k = (torch.randn(1, 1, n, 128).to(torch.bfloat16).cuda() for _ in range(2))
    _assert_same(*_both(q, k, 2048, seed=2))


def test_fused_plan_exact_probe_path():
    """With kept prefixes, a row whose thresholds could land in a rounding drop
    of the prefix array makes the reference's probes instead of the two-level
    search; ab_ibcs_sip_exact_draws takes that path for every row and must
    give the same bits as ab_ibcs_sip and as _C.ibcs then _C.sip."""
    print("fused plan forced reference probes n=108000", flush=True)
    torch.manual_seed(9)
    n, samples = 108000, 2048
    q, k = (torch.randn(1, 2, n, 128).to(torch.bfloat16).cuda() for _ in range(2))
    ids_f, w_f, ids_s, w_s = _both(q, k, samples, seed=4)
    _assert_same(ids_f, w_f, ids_s, w_s)
    rows = ids_f.shape[0]
    offsets = torch.rand(rows, generator=torch.Generator().manual_seed(4)).cuda()
    ids_x = torch.empty_like(ids_f)
    w_x = torch.empty_like(w_f)
    lib = _lib.load()
    ws_bytes = lib.ab_ibcs_sip_workspace_bytes(2, n)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    _lib.check(lib.ab_ibcs_sip_exact_draws(_lib.ptr(q), _lib.ptr(k), None, 2, n, _lib.ptr(offsets), samples,
                                           _lib.ptr(workspace), ws_bytes, _lib.ptr(ids_x), _lib.ptr(w_x),
                                           _lib.stream(q.device)))
    torch.cuda.synchronize()
    _assert_same(ids_x, w_x, ids_s, w_s)


def test_build_plan_uses_fused_path():
    """build_plan's plan equals the reference-structured path's on the same uniforms."""
    print("build_plan vs ibcs+sip", flush=True)
    q, k, _ = make_qkv(CONFIGS[0], dtype=torch.bfloat16)
    q, k = q.cuda(), k.cuda()
    plan = build_plan(q, k, sample_pages=2, seed=42)
    rows = plan.descriptor.shape[0]
    offsets = torch.rand(rows, device=q.device, generator=torch.Generator(q.device).manual_seed(42))
    ids = torch.empty(rows, 64, dtype=torch.int32, device=q.device)
    w = torch.empty(rows, 64, dtype=torch.float32, device=q.device)
    _C.sip(_C.ibcs(q, k), offsets, ids, w)
    torch.cuda.synchronize()
    _assert_same(plan.descriptor.reshape(rows, 64), plan.log_weights.reshape(rows, 64), ids, w)


def test_build_plan_independent_of_head_chunks(monkeypatch):
    """Lowering the IBCS budget to one head per chunk (one native call per
    head) leaves the plan bit-identical: the uniforms are drawn first."""
    from ab_attention import attention

    print("build_plan chunking", flush=True)
    torch.manual_seed(12)
    q, k = (torch.randn(2, 3, 4096, 128).to(torch.bfloat16).cuda() for _ in range(2))
    whole = build_plan(q, k, sample_pages=4, seed=3)
    monkeypatch.setattr(attention, "LSE_BUDGET_BYTES", 1)
    chunked = build_plan(q, k, sample_pages=4, seed=3)
    torch.cuda.synchronize()
    _assert_same(whole.descriptor, whole.log_weights, chunked.descriptor, chunked.log_weights)


@pytest.mark.parametrize("n,samples", [(2048, 64), (108000, 2048)])
def test_fused_plan_with_certainty(oracle_mod, n, samples):
    """Rows with certain blocks (pi = 1: weight 0, listed first), through the
    full prefix array (2,048 tokens) and the kept prefixes (108,000): queries
    share a direction and three KV4 blocks per head hold keys along it, so each
    of those blocks takes about a third of every row's mass. The certainty
    passes, the certain ids and the draws of the remaining mass must give the
    same bits as _C.ibcs then _C.sip (the synthetic configs have no certain
    blocks), and the oracle's SIP on the GPU's scores."""
    print(f"fused plan with certainty n={n} samples={samples}", flush=True)
    torch.manual_seed(11)
    q = (torch.randn(1, 2, n, 128) + 1.0).to(torch.bfloat16)
    k = torch.randn(1, 2, n, 128)
    hot = [10, 100, 300]
    for j in hot:
        k[:, :, 4 * j:4 * j + 4] = 3.0
    k = k.to(torch.bfloat16)
    ids_f, w_f, ids_s, w_s = _both(q.cuda(), k.cuda(), samples, seed=6)
    _assert_same(ids_f, w_f, ids_s, w_s)
    certain = (w_f == 0).sum(dim=1)
    assert bool((certain >= len(hot)).all()), certain.min().item()
    assert torch.equal(ids_f[:, :len(hot)].cpu(), torch.tensor(hot, dtype=torch.int32).expand(ids_f.shape[0], -1))
    rows = ids_f.shape[0]
    offsets = torch.rand(rows, generator=torch.Generator().manual_seed(6))
    scores = _C.ibcs(q.cuda(), k.cuda()).cpu().numpy()
    ids_o, w_o = oracle_mod.sip(scores, offsets.numpy(), samples)
    assert (ids_f.cpu().numpy() == ids_o).all()
    assert (w_f.cpu().numpy().view("uint32") == w_o.view("uint32")).all()
