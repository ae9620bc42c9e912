"""fp8 scales stored as (K, V) pairs per (page, kv-head) (kv_cache.
paired_scales: v_scale == k_scale + 1, one cache line per page's two scales)
against two separate arrays of the same values: decode outputs (MFMA with
d-major and token-major V, VALU, linear mode, split tiles) and the writer's
pools and regrown scales are bitwise equal; and the oracle on the result."""
import numpy as np
import pytest
import torch

import oracle
import sched_abi as abi
import sched_pd
from kv_cache import append as kv_append
from kv_cache import paired_scales
from parity import TOL_BF16, par_err

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


@pytest.fixture(scope="module", autouse=True)
def lib(schedlib):
    torch.cuda.init()
    return schedlib


def batch(v_layout, seed=0, lens=(1, 17, 300, 1000, 64, 2049), hq=28, hkv=4, d=128, ps=16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    npg = [-(-n // ps) for n in lens]
    P = sum(npg) + 3
    k = (torch.randn(P, hkv, ps, d, device="cuda", generator=g) * 8).to(FP8)
    vshape = (P, hkv, d, ps) if v_layout == "dmajor" else (P, hkv, ps, d)
    v = (torch.randn(*vshape, device="cuda", generator=g) * 8).to(FP8)
    ks = torch.rand(P * hkv, device="cuda", generator=g) * 0.09 + 0.01
    vs = torch.rand(P * hkv, device="cuda", generator=g) * 0.09 + 0.01
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(seed)).numpy()
    bt = np.zeros((len(lens), max(npg)), np.int32)
    off = 0
    for r, n in enumerate(npg):
        bt[r, :n] = perm[off:off + n]
        off += n
    q = (torch.randn(len(lens), hq, d, device="cuda", generator=g) / d ** 0.5).bfloat16()
    return dict(q=q, k=k, v=v, ks=ks, vs=vs, bt=torch.from_numpy(bt).cuda(),
                ctx=torch.tensor(lens, dtype=torch.int32, device="cuda"), hkv=hkv)


def paired(ks, vs):
    kp, vp = paired_scales(ks.numel(), ks.device)
    kp.copy_(ks)
    vp.copy_(vs)
    assert vp.data_ptr() == kp.data_ptr() + 4
    return kp, vp


@pytest.mark.parametrize("v_layout", ["dmajor", "tokmajor"])
@pytest.mark.parametrize("variant", ["mfma", "valu", "linear", "tiles"])
def test_decode_bits_do_not_depend_on_the_scale_layout(v_layout, variant):
    b = batch(v_layout, seed=3)
    kp, vp = paired(b["ks"], b["vs"])
    kw = dict(v_layout=v_layout)
    mode = abi.SOFTMAX
    if variant == "valu":
        kw["flags"] = abi.FLAG_FORCE_VALU
    elif variant == "linear":
        mode = abi.LINEAR
        kw["lin_w"] = torch.randn(4096, device="cuda")
    elif variant == "tiles":
        kw["tiles"] = sched_pd.plan_tiles_host(b["ctx"].cpu().numpy(), 16, 8, b["hkv"])
        kw["tile_pages"] = 8
    outs = []
    for ks, vs in ((b["ks"], b["vs"]), (kp, vp)):
        outs.append(sched_pd.paged_decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"],
                                          k_scale=ks, v_scale=vs, mode=mode,
                                          out_dtype=torch.float32, **kw))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    if variant in ("mfma", "tiles"):
        ref = oracle.decode(b["q"], b["k"], b["v"], b["bt"], b["ctx"], v_layout=v_layout,
                            k_scale=b["ks"], v_scale=b["vs"])
        assert par_err(outs[1].cpu(), ref) <= TOL_BF16


@pytest.mark.parametrize("v_layout", ["dmajor", "tokmajor"])
def test_writer_pools_and_regrown_scales_do_not_depend_on_the_scale_layout(v_layout):
    """Two appends per request, the second with larger values, so scales
    regrow and earlier codes are re-encoded; both layouts end equal, and
    equal the oracle's writer."""
    hkv, d, ps = 4, 128, 16
    lens0, lens1 = [5, 16, 40, 33], [3, 20, 8, 31]
    R = len(lens0)
    npg = [-(-(a + b_) // ps) for a, b_ in zip(lens0, lens1)]
    P = sum(npg) + 2
    bt = np.zeros((R, max(npg)), np.int32)
    off = 0
    for r, n in enumerate(npg):
        bt[r, :n] = np.arange(off, off + n)[::-1]
        off += n
    bt = torch.from_numpy(bt).cuda()
    g = torch.Generator(device="cuda").manual_seed(5)
    vshape = (P, hkv, d, ps) if v_layout == "dmajor" else (P, hkv, ps, d)
    pools = []
    for layout in ("separate", "pairs"):
        k = torch.zeros(P, hkv, ps, d, dtype=FP8, device="cuda")
        v = torch.zeros(*vshape, dtype=FP8, device="cuda")
        if layout == "separate":
            ks = torch.zeros(P * hkv, device="cuda")
            vs = torch.zeros(P * hkv, device="cuda")
        else:
            ks, vs = paired_scales(P * hkv, "cuda")
        pools.append((k, v, ks, vs))
    srcs = []
    for step, (lens, amp) in enumerate(((lens0, 1.0), (lens1, 50.0))):
        T = sum(lens)
        gs = torch.Generator(device="cuda").manual_seed(11 + step)
        ksrc = torch.randn(T, hkv, d, device="cuda", generator=gs) * amp
        vsrc = torch.randn(T, hkv, d, device="cuda", generator=gs) * amp
        ind = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32,
                           device="cuda")
        done = lens0 if step == 1 else [0] * R
        ctx = torch.tensor([a + b_ for a, b_ in zip(done, lens)], dtype=torch.int32,
                           device="cuda")
        srcs.append((ksrc, vsrc, ind, ctx))
        for k, v, ks, vs in pools:
            kv_append(ksrc, vsrc, ind, ctx, k, v, bt, v_layout=v_layout, k_scale=ks,
                      v_scale=vs, max_append=max(lens))
    torch.cuda.synchronize()
    (k0, v0, ks0, vs0), (k1, v1, ks1, vs1) = pools
    assert torch.equal(k0.view(torch.uint8), k1.view(torch.uint8))
    assert torch.equal(v0.view(torch.uint8), v1.view(torch.uint8))
    assert torch.equal(ks0, ks1) and torch.equal(vs0, vs1)
    assert (ks1 > 0).any()
    # the oracle's writer, replayed on the host over the same two appends
    hk = torch.zeros(P, hkv, ps, d, dtype=FP8)
    hv = torch.zeros(*vshape, dtype=FP8)
    hks = np.zeros(P * hkv, np.float32)
    hvs = np.zeros(P * hkv, np.float32)
    for ksrc, vsrc, ind, ctx in srcs:
        k_, v_, hks, hvs, _ = oracle.kv_append(ksrc, vsrc, ind, ctx, hk, hv, bt,
                                               v_layout=v_layout, k_scale=hks, v_scale=hvs)
        hk = torch.from_numpy(k_).view(FP8)
        hv = torch.from_numpy(v_).view(FP8)
    hk, hv = hk.view(torch.uint8).numpy(), hv.view(torch.uint8).numpy()
    assert np.array_equal(hk, k1.view(torch.uint8).cpu().numpy())
    assert np.array_equal(hv, v1.view(torch.uint8).cpu().numpy())
    assert np.array_equal(hks, ks1.cpu().numpy()) and np.array_equal(hvs, vs1.cpu().numpy())
