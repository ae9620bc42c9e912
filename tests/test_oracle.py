"""Pins the oracle (CPU only): dequantisation against torch's own types, the C
restatement against an independent numpy closed form, closed-form special
cases, and planted mistakes that the checks must catch."""
import numpy as np
import pytest
import torch

import oracle
import sched_abi as abi

F64, F32 = oracle.F64, oracle.F32


def mixed_close(a, r, tol):
    """|a - r| <= tol * (1 + |r|) elementwise (test/paged_decode.cu:268-274)."""
    a, r = np.asarray(a, np.float64), np.asarray(r, np.float64)
    return bool(np.all(np.abs(a - r) <= tol * (1 + np.abs(r))))


def small_batch(ctx, hq, hkv, d, dtype, seed=0, ps=16, extra_pages=3):
    b = {}
    g = torch.Generator().manual_seed(seed)
    ctx = np.asarray(ctx, np.int32)
    npg = (ctx + ps - 1) // ps
    P = int(npg.sum()) + extra_pages
    scale = 1.0 if dtype == torch.float32 else 0.3
    b["q"] = (torch.randn(len(ctx), hq, d, generator=g) * scale).to(
        torch.float32 if dtype == torch.float32 else torch.bfloat16)
    b["k"] = (torch.randn(P, hkv, ps, d, generator=g) * scale).to(dtype)
    b["v"] = (torch.randn(P, hkv, d, ps, generator=g) * scale).to(dtype)
    if dtype == torch.float8_e4m3fn:
        b["ks"] = torch.rand(P, hkv, generator=g) * 0.09 + 0.01
        b["vs"] = torch.rand(P, hkv, generator=g) * 0.09 + 0.01
    else:
        b["ks"] = b["vs"] = None
    perm = torch.randperm(P, generator=g).numpy().astype(np.int32)
    bt = np.zeros((len(ctx), max(int(npg.max()), 1)), np.int32)
    off = 0
    for r in range(len(ctx)):
        bt[r, :npg[r]] = perm[off:off + npg[r]]
        off += npg[r]
    b["bt"], b["ctx"], b["ps"] = bt, ctx, ps
    return b


def run_both(b, tau=None, tau_scope=abi.TAU_PREFIX, mode=abi.SOFTMAX, lin_w=None,
             period=0, max_tasks=4096):
    hkv = b["v"].shape[1]
    ctrl = None
    if tau is not None:
        import levers
        ctrl = levers.ctrl_bytes({"rows": {t: (0.0, int(x), 0) for t, x in enumerate(tau)}},
                                 max_tasks)
    c = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"], mode=mode,
                      k_scale=b["ks"], v_scale=b["vs"], tau_scope=tau_scope,
                      lin_w=lin_w, lin_w_period=period, ctrl=ctrl, max_tasks=max_tasks)
    n = oracle.numpy_decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"], mode=mode,
                            k_scale=b["ks"], v_scale=b["vs"], tau=tau, tau_scope=tau_scope,
                            lin_w=lin_w, lin_w_period=period)
    return c, n


# --- dequantisation ----------------------------------------------------------

def test_fp8_e4m3fn_table_matches_torch_all_256_codes():
    ours = oracle.fp8_e4m3_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert nan.sum() == 2  # 0x7f and 0xff only: no infinity in e4m3fn
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_decode_matches_torch_on_every_code():
    """The oracle's binary16 decode (from the format definition) against
    torch's on all 65536 codes: subnormals, infinities, every exponent."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.float16).float().numpy()
    lib = oracle.load()
    ours = np.array([lib.oracle_f16_to_float(int(x)) for x in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # the closed forms the decode follows: smallest subnormal, largest finite
    assert ours[1] == 2.0 ** -24 and ours[0x7bff] == 65504.0 and ours[0x3c00] == 1.0


def test_bf16_decode_matches_torch():
    bits = np.random.default_rng(0).integers(0, 1 << 16, 4096, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7f80) != 0x7f80]  # finite values
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    lib = oracle.load()
    ours = np.array([lib.oracle_bf16_to_float(int(x)) for x in bits], np.float32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(oracle.bf16_to_float(bits).view(np.uint32), ref.view(np.uint32))


# --- C restatement vs numpy closed form ---------------------------------------

CASES = [
    # ctx, hq, hkv, d, dtype
    ([64, 100, 7, 512, 33], 8, 8, 64, torch.float32),      # MHA fp32, partial pages
    ([48, 130, 17], 32, 8, 128, torch.bfloat16),           # GQA-4 bf16
    ([16, 200, 5], 28, 4, 128, torch.float8_e4m3fn),       # GQA-7 fp8 + scales
    ([40, 9], 4, 1, 32, torch.float32),                    # d 32
]


@pytest.mark.parametrize("ctx,hq,hkv,d,dtype", CASES)
@pytest.mark.parametrize("shed", ["none", "prefix", "per_page"])
def test_c_oracle_matches_numpy_closed_form(ctx, hq, hkv, d, dtype, shed):
    b = small_batch(ctx, hq, hkv, d, dtype, seed=len(ctx) + d)
    tau, scope = None, abi.TAU_PREFIX
    if shed != "none":
        rng = np.random.default_rng(1)
        tau = [int(rng.integers(1, 40)) for _ in range(len(ctx) * hkv)]
        scope = abi.TAU_PREFIX if shed == "prefix" else abi.TAU_PER_PAGE
    c, n = run_both(b, tau, scope)
    assert np.allclose(c, n, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("period", [0, 16])
def test_linear_matches_numpy(dtype, period):
    b = small_batch([70, 16, 3], 2, 2, 64, dtype, seed=5)
    w = np.random.default_rng(2).standard_normal(128).astype(np.float32)
    tau = [0, 5, 9, 2, 40, 1]
    c, n = run_both(b, tau, abi.TAU_PREFIX, mode=abi.LINEAR, lin_w=w, period=period)
    assert np.allclose(c, n, rtol=1e-12, atol=1e-12)


def test_csr_page_table_equals_2d_table():
    b = small_batch([70, 16, 33], 4, 2, 64, torch.float32, seed=9)
    npg = (b["ctx"] + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(npg)]).astype(np.int32)
    flat = np.concatenate([b["bt"][r, :npg[r]] for r in range(3)]).astype(np.int32)
    a = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"])
    c = oracle.decode(b["q"], b["k"], b["v"], flat, b["ctx"], page_indptr=indptr)
    assert np.array_equal(a, c)


# --- closed-form special cases -----------------------------------------------

def test_tau_one_prefix_returns_first_value_exactly():
    b = small_batch([50, 33], 8, 2, 64, torch.float32, seed=3)
    c, _ = run_both(b, tau=[1] * 4)
    V = b["v"].numpy()
    for r in range(2):
        for hq in range(8):
            h = hq // 4
            assert np.array_equal(c[r, hq], V[b["bt"][r, 0], h, :, 0].astype(np.float64))


def test_context_one_returns_its_value():
    b = small_batch([1, 1], 4, 4, 64, torch.float32, seed=4)
    c, _ = run_both(b)
    V = b["v"].numpy()
    for r in range(2):
        for h in range(4):
            assert np.array_equal(c[r, h], V[b["bt"][r, 0], h, :, 0].astype(np.float64))


def test_zero_query_gives_mean_of_kept_values():
    b = small_batch([37, 64], 4, 2, 64, torch.float32, seed=6)
    b["q"] = torch.zeros_like(b["q"])
    tau = [0, 0, 20, 5]
    c, _ = run_both(b, tau=tau)
    V = b["v"].numpy().astype(np.float64)
    for r in range(2):
        for h in range(2):
            n = int(b["ctx"][r])
            t = tau[r * 2 + h]
            keep = np.arange(n) if t == 0 else np.arange(min(n, t))
            vals = np.stack([V[b["bt"][r, p // 16], h, :, p % 16] for p in keep])
            for g in range(2):
                assert np.allclose(c[r, h * 2 + g], vals.mean(0), rtol=1e-12, atol=1e-14)


def test_dominant_score_selects_its_value():
    b = small_batch([40], 1, 1, 64, torch.float32, seed=7)
    qv = b["q"][0, 0].clone()
    page, i = b["bt"][0, 1], 5          # token 21
    b["k"][page, 0, i] = qv * 50.0      # score ~ 50 |q|^2 / 8, far above the rest
    c, _ = run_both(b)
    assert np.allclose(c[0, 0], b["v"][page, 0, :, i].numpy(), rtol=0, atol=1e-6)


def test_tau_at_least_context_is_full_attention_bitwise():
    b = small_batch([30, 47], 4, 2, 64, torch.float32, seed=8)
    full, _ = run_both(b)
    cap, _ = run_both(b, tau=[47, 47, 60, 60])
    assert np.array_equal(full, cap)


def test_empty_request_is_nan_like_reference_zero_over_zero():
    b = small_batch([0, 16], 2, 2, 64, torch.float32, seed=10)
    c, n = run_both(b)
    assert np.isnan(c[0]).all() and np.isnan(n[0]).all()
    assert np.isfinite(c[1]).all()


def test_page_relocation_is_invisible():
    b = small_batch([70, 33], 4, 2, 64, torch.bfloat16, seed=11)
    a = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"])
    P = b["k"].shape[0]
    perm = np.random.default_rng(0).permutation(P)
    inv = np.argsort(perm)
    k2, v2 = b["k"][torch.from_numpy(perm)], b["v"][torch.from_numpy(perm)]
    bt2 = inv[b["bt"]].astype(np.int32)
    c = oracle.decode(b["q"], k2, v2, bt2, b["ctx"])
    assert np.array_equal(a, c)


def test_f32_port_matches_f64_expected_values():
    b = small_batch([512, 300, 64], 8, 8, 64, torch.float32, seed=12)
    f64 = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"], precision=F64)
    f32 = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"], precision=F32)
    assert mixed_close(f32, f64, 1e-5)


# --- planted mistakes: each must be caught by the comparisons above ----------

def test_planted_mistakes_are_caught():
    # transposed V operand (page 32 = d 32, so the swap is shape-compatible)
    sq = small_batch([70, 33], 4, 2, 32, torch.float32, seed=14, ps=32)
    good = oracle.numpy_decode(sq["q"], sq["k"], sq["v"], sq["bt"], sq["ctx"])
    assert np.allclose(oracle.decode(sq["q"], sq["k"], sq["v"], sq["bt"], sq["ctx"]), good,
                       rtol=1e-12, atol=1e-12)
    bad = oracle.decode(sq["q"], sq["k"], sq["v"].transpose(2, 3), sq["bt"], sq["ctx"])
    assert not np.allclose(bad, good, atol=1e-6)

    b = small_batch([70, 33], 8, 2, 64, torch.float32, seed=13)
    good = oracle.numpy_decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"])
    # wrong sign of the scale
    bad = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"], sm_scale=-0.125)
    assert not np.allclose(bad, good, atol=1e-6)
    # dropped last token
    bad = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"] - 1)
    assert not np.allclose(bad, good, atol=1e-6)
    # wrong page index (off by one in the table)
    bad = oracle.decode(b["q"], b["k"], b["v"], (b["bt"] + 1) % b["k"].shape[0], b["ctx"])
    assert not np.allclose(bad, good, atol=1e-6)


# --- the reference fixture's own inputs (test/paged_decode.cu:236-251) -------

def lcg_fixture(nseq=64, nblocks=8, page_tokens=64, sd=32, seed=12345):
    """The fixture's LCG stream and page map, restated: kv, w, then q."""
    npages = nseq * nblocks
    n_kv = npages * page_tokens * 2 * sd
    s = np.uint64(seed)
    out = np.empty(n_kv + nblocks * page_tokens + nseq * sd, np.float32)
    st = int(seed)
    for i in range(out.size):
        st = (st * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = ((st >> 8) & 0xFFFF) / 65536.0 - 0.5
    kv = out[:n_kv]
    q = out[n_kv + nblocks * page_tokens:]
    bt = np.array([(i * 37 + 11) % npages for i in range(nseq * nblocks)], np.int32)
    return kv, bt.reshape(nseq, nblocks), q.reshape(nseq, 1, sd)


def test_reference_fixture_layout_per_page_tau():
    kv, bt, q = lcg_fixture(nseq=8, nblocks=3, page_tokens=64)
    P = kv.size // (64 * 64)
    pages = kv.reshape(P, 64, 64)                     # [page][token][K|V]
    k = pages[:, None, :, :32]                        # [P, 1, 64, 32] (strided view)
    v = pages[:, None, :, 32:].transpose(0, 1, 3, 2)  # [P, 1, 32, 64] d-major view
    ctx = np.full(8, 3, np.int32)                     # pages
    for tau in (0, 8):
        import levers
        ctrl = levers.ctrl_bytes({"rows": {t: (0.0, tau, 0) for t in range(8)}}, 64)
        c = oracle.decode(q, np.ascontiguousarray(k), np.ascontiguousarray(v), bt, ctx,
                          sm_scale=0.125, tau_scope=abi.TAU_PER_PAGE, ctrl=ctrl,
                          max_tasks=64, ctx_in_pages=True)
        n = oracle.numpy_decode(q, np.ascontiguousarray(k), np.ascontiguousarray(v), bt,
                                ctx * 64, sm_scale=0.125, tau=[tau] * 8,
                                tau_scope=abi.TAU_PER_PAGE)
        assert np.allclose(c, n, rtol=1e-12, atol=1e-12)
