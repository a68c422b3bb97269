"""The Python surface keeps the reference's names, defaults and validation
(ab_attention/attention.py:26-102, flashinfer_backend.py:164-193; the native
op checks of csrc/ibcs.cu:550-568 and csrc/sip.cu:172-192). CPU only: every
check here fires before any launch."""
import inspect

import pytest
import torch

import ab_attention
from ab_attention import SamplePlan, _C, ab_attention as ab_attn, apply_plan, build_plan
from ab_attention.flashinfer_backend import paged_attention


def test_public_names_and_defaults():
    assert ab_attention.__all__ == ["SamplePlan", "ab_attention", "apply_plan", "build_plan"]
    assert SamplePlan._fields == ("descriptor", "log_weights")
    sig = inspect.signature(build_plan)
    assert sig.parameters["sample_pages"].default == 64 and sig.parameters["seed"].default == 42
    assert inspect.signature(apply_plan).parameters["return_lse"].default is False
    assert inspect.signature(ab_attn).parameters["sample_pages"].default == 64
    assert inspect.signature(paged_attention).parameters["return_lse"].default is False


def _qk(shape=(1, 2, 1024, 128), dtype=torch.bfloat16):
    return torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)


@pytest.mark.parametrize("shape_q,shape_k,pages,msg", [
    ((2, 1024, 128), (2, 1024, 128), 1, "N divisible by 4"),
    ((1, 2, 1024, 128), (1, 2, 1020, 128), 1, "N divisible by 4"),
    ((1, 2, 1022, 128), (1, 2, 1022, 128), 1, "N divisible by 4"),
    ((1, 2, 1024, 128), (1, 2, 1024, 128), 0, "positive"),
    ((1, 2, 1024, 128), (1, 2, 1024, 128), 8, "smaller than the sequence"),
])
def test_build_plan_value_errors(shape_q, shape_k, pages, msg):
    with pytest.raises(ValueError, match=msg):
        build_plan(torch.zeros(shape_q, dtype=torch.bfloat16), torch.zeros(shape_k, dtype=torch.bfloat16),
                   sample_pages=pages)


def test_build_plan_rejects_cpu_tensors_in_native_op():
    q, k = _qk()
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        build_plan(q, k, sample_pages=2)


def test_native_op_checks():
    q, k = _qk()
    with pytest.raises(RuntimeError, match="CUDA"):
        _C.ibcs(q, k)
    s = torch.zeros(4, 16)
    with pytest.raises(RuntimeError, match="CUDA"):
        _C.sip(s, torch.zeros(4), torch.zeros(4, 2, dtype=torch.int32), torch.zeros(4, 2))


def test_paged_attention_value_errors():
    q = torch.zeros(1, 2, 512, 128, dtype=torch.bfloat16)
    rows = 2 * 4
    desc = torch.zeros(rows, 1, 32, dtype=torch.int32)
    w = torch.zeros(rows, 1, 32)
    with pytest.raises(ValueError, match="same"):
        paged_attention(q, q[:, :1], q, desc, w)
    with pytest.raises(ValueError, match="GPU"):
        paged_attention(q, q, q, desc, w)



def test_apply_plan_forwards_validation():
    q = torch.zeros(1, 1, 256, 128, dtype=torch.bfloat16)
    plan = SamplePlan(torch.zeros(3, 1, 32, dtype=torch.int32), torch.zeros(3, 1, 32))
    with pytest.raises(ValueError):
        apply_plan(q, q, q, plan)


def test_heads_per_chunk_budget():
    from ab_attention.attention import _heads_per_chunk

    # Wan2.1-14B 720p runs as one chunk within the 16 GiB budget
    assert _heads_per_chunk(80, 591, 75600) == 80
    assert _heads_per_chunk(4, 10, 1280) == 4


def test_dense_page_list_padding():
    """Dense page lists (exact attention, Hunyuan prompt blocks): every block
    once at weight 0, padded to a multiple of 8 with removed (-inf) repeats."""
    import torch
    from ab_attention.video import _dense_pages

    ids, w = _dense_pages(3, 10, "cpu", offset=5)
    assert ids.shape == (3, 16) and w.shape == (3, 16)
    assert ids[0, :10].tolist() == list(range(5, 15)) and ids[0, 10:].tolist() == [5] * 6
    assert torch.all(w[:, :10] == 0) and torch.all(torch.isinf(w[:, 10:])) and torch.all(w[:, 10:] < 0)
    assert torch.equal(ids[2], ids[0])
    ids, w = _dense_pages(1, 64, "cpu")
    assert ids.shape == (1, 64) and torch.all(w == 0)


def test_video_validation_errors():
    import pytest
    import torch
    from ab_attention.video import VideoAttention, exact_attention, hunyuan_attention, merge_states

    q = torch.zeros(1, 2, 64, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        exact_attention(q, q[:, :, :62], q[:, :, :62])  # K/V length not divisible by 4
    with pytest.raises(ValueError):
        exact_attention(q, q, q)  # CPU tensors
    with pytest.raises(ValueError):
        hunyuan_attention(VideoAttention(1), 1, q, q, q, 30, 32)  # video length not divisible by 4
    with pytest.raises(ValueError):
        merge_states((q, torch.zeros(1, 2, 64)), (q, torch.zeros(1, 2, 63)))
    sched = VideoAttention(4)
    assert not sched.is_sparse(1)
    sched.step = 11
    assert sched.is_sparse(1) and not sched.is_sparse(0)
    assert not VideoAttention(4, dense=True).is_sparse(3)


def test_lse_budget_sets_head_chunks(monkeypatch):
    """LSE_BUDGET_BYTES bounds the pair-LSE bytes of one head chunk (at least
    one head per chunk); the reference's 1.5 GiB gives its nine chunks of at
    most 9 heads at Wan2.1-14B 720p (attention.py:8, :61-64)."""
    from ab_attention import attention

    per_head = 591 * 8 * 18900 * 2
    monkeypatch.setattr(attention, "LSE_BUDGET_BYTES", int(1.5 * 1024 ** 3))
    assert attention._heads_per_chunk(80, 591, 75600) == 9
    monkeypatch.setattr(attention, "LSE_BUDGET_BYTES", per_head - 1)
    assert attention._heads_per_chunk(80, 591, 75600) == 1
    monkeypatch.setattr(attention, "LSE_BUDGET_BYTES", 16 * 1024 ** 3)
    assert attention._heads_per_chunk(80, 591, 75600) == 80


def test_compact_plan_round_trip():
    """int16 plan ids are exact for every id a head can have (0..32,767)."""
    import torch
    from ab_attention import SamplePlan
    from ab_attention.video import compact_plan, expand_plan

    ids = torch.arange(0, 32768, dtype=torch.int32).reshape(32, 32, 32)
    w = torch.rand(32, 32, 32)
    c = compact_plan(SamplePlan(ids, w))
    assert c.descriptor.dtype == torch.int16 and c.descriptor.element_size() == 2
    back = expand_plan(c)
    assert back.descriptor.dtype == torch.int32 and torch.equal(back.descriptor, ids)
    assert torch.equal(back.log_weights, w)


def test_lse_budget_env_parsing(monkeypatch):
    """AB_ATTENTION_LSE_BUDGET_BYTES takes an integer or a float byte count;
    anything else raises a ValueError that names the variable."""
    from ab_attention import attention

    monkeypatch.delenv("AB_ATTENTION_LSE_BUDGET_BYTES", raising=False)
    assert attention._budget_from_env(123) == 123
    for raw, want in (("1610612736", 1610612736), ("1.5e9", 1500000000), (" 2048 ", 2048)):
        monkeypatch.setenv("AB_ATTENTION_LSE_BUDGET_BYTES", raw)
        assert attention._budget_from_env(123) == want
    for raw in ("1.5GiB", "-1", "0", "nan", "inf"):
        monkeypatch.setenv("AB_ATTENTION_LSE_BUDGET_BYTES", raw)
        with pytest.raises(ValueError, match="AB_ATTENTION_LSE_BUDGET_BYTES"):
            attention._budget_from_env(123)
