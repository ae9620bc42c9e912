"""The FlashInfer wrapper's plan() / run() argument handling without a GPU:
the CSR table becomes per-request token counts, dtypes are taken as FlashInfer
takes them (torch dtypes or names, kv_data_type as an alias of data_type),
and every option that would change the arithmetic is rejected, as are shapes
and dtypes that differ from the plan (before anything is launched)."""
import pytest
import torch

from flashinfer_compat import BatchDecodeWithPagedKVCacheWrapper


def table():
    indptr = torch.tensor([0, 3, 4, 9], dtype=torch.int32)
    indices = torch.arange(9, dtype=torch.int32)
    last = torch.tensor([16, 1, 7], dtype=torch.int32)
    return indptr, indices, last


def test_plan_turns_the_csr_table_into_token_counts():
    w = BatchDecodeWithPagedKVCacheWrapper(None, "NHD")
    w.plan(*table(), 16, 2, 128, 16, data_type=torch.float16, q_data_type=torch.float16)
    p = w._plan
    assert p["ctx"].tolist() == [2 * 16 + 16, 1, 4 * 16 + 7]
    assert (p["hq"], p["hkv"], p["d"], p["page"]) == (16, 2, 128, 16)
    assert p["kv_dtype"] == torch.float16 and p["q_dtype"] == torch.float16


@pytest.mark.parametrize("kw,kv,q", [
    (dict(), torch.float16, torch.float16),
    (dict(data_type="bfloat16"), torch.bfloat16, torch.bfloat16),
    (dict(kv_data_type=torch.bfloat16, q_data_type="float16"), torch.bfloat16, torch.float16),
    (dict(data_type="torch.float16", kv_data_type=torch.float16), torch.float16, torch.float16),
])
def test_plan_dtypes(kw, kv, q):
    w = BatchDecodeWithPagedKVCacheWrapper(None, "HND")
    w.plan(*table(), 8, 8, 64, 16, **kw)
    assert w._plan["kv_dtype"] == kv and w._plan["q_dtype"] == q


@pytest.mark.parametrize("kw,msg", [
    (dict(pos_encoding_mode="ROPE_LLAMA"), "positional"),
    (dict(window_left=128), "window"),
    (dict(logits_soft_cap=30.0), "soft cap"),
    (dict(data_type=torch.float16, kv_data_type=torch.bfloat16), "differ"),
    (dict(data_type="float17"), "unknown dtype"),
])
def test_plan_rejects(kw, msg):
    w = BatchDecodeWithPagedKVCacheWrapper(None, "NHD")
    with pytest.raises(ValueError, match=msg):
        w.plan(*table(), 8, 8, 64, 16, **kw)


def test_plan_checks_heads_and_index_dtypes():
    w = BatchDecodeWithPagedKVCacheWrapper(None, "NHD")
    with pytest.raises(ValueError, match="multiple"):
        w.plan(*table(), 12, 8, 64, 16)
    indptr, indices, last = table()
    with pytest.raises(ValueError, match="int32"):
        w.plan(indptr.long(), indices, last, 8, 8, 64, 16)
    with pytest.raises(ValueError, match="NHD or HND"):
        BatchDecodeWithPagedKVCacheWrapper(None, "HDN")


def test_run_checks_the_plan_before_launching():
    w = BatchDecodeWithPagedKVCacheWrapper(None, "NHD")
    kv = torch.zeros(9, 2, 16, 2, 128, dtype=torch.float16)
    q = torch.zeros(3, 16, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="plan"):
        w.run(q, kv)
    w.plan(*table(), 16, 2, 128, 16)
    with pytest.raises(ValueError, match="do not match"):
        w.run(q, torch.zeros(9, 2, 16, 4, 128, dtype=torch.float16))
    with pytest.raises(ValueError, match="dtypes"):
        w.run(q.bfloat16(), kv)
    with pytest.raises(ValueError, match="paged cache"):
        w.run(q, kv[:, 0])
    with pytest.raises(ValueError, match="fp8 caches only"):
        w.run(q, kv, k_scale=0.5)
