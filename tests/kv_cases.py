"""Append cases shared by the CPU and GPU writer tests: seeded inputs on the
host, the oracle's result, and readback through the page table."""
import numpy as np
import torch

import oracle

FP8 = torch.float8_e4m3fn


def fp8_values() -> np.ndarray:
    return oracle.fp8_e4m3_table()


def random_pool(shape, dtype, rng):
    if dtype == FP8:
        codes = rng.integers(0, 0x7e, size=shape, dtype=np.uint8)   # finite codes only
        codes |= rng.integers(0, 2, size=shape, dtype=np.uint8) << 7
        return torch.from_numpy(codes).view(FP8)
    bits = rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)
    if dtype == torch.bfloat16:
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    if dtype == torch.float16:
        return torch.from_numpy(bits.view(np.int16)).view(torch.float16)
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32))


def append_case(seed, kv_dtype, v_layout="dmajor", csr=False, prior=None, hkv=2, d=16, ps=16,
                n=None, src_dtype=torch.bfloat16):
    """A batch appending n[r] rows on top of prior[r] tokens. Returns the
    inputs and the oracle's outputs."""
    rng = np.random.default_rng(seed)
    R = 5
    prior = rng.integers(0, 40, R) if prior is None else np.asarray(prior)
    n = rng.integers(0, 30, R) if n is None else np.asarray(n)
    ctx = prior + n
    pages_per = -(-ctx // ps)
    P = int(pages_per.sum()) + 7
    perm = rng.permutation(P).astype(np.int32)
    app = np.zeros(R + 1, np.int32)
    app[1:] = np.cumsum(n)
    T = int(app[-1])
    k_src = torch.from_numpy(rng.standard_normal((T, hkv, d)).astype(np.float32)).to(src_dtype)
    v_src = torch.from_numpy(rng.standard_normal((T, hkv, d)).astype(np.float32) * 3).to(src_dtype)
    k_pool = random_pool((P, hkv, ps, d), kv_dtype, rng)
    v_pool = random_pool((P, hkv, d, ps) if v_layout == "dmajor" else (P, hkv, ps, d), kv_dtype, rng)
    ks = vs = None
    if kv_dtype == FP8:
        ks = torch.from_numpy(np.exp2(rng.integers(-8, 2, P * hkv)).astype(np.float32))
        vs = torch.from_numpy(np.exp2(rng.integers(-8, 2, P * hkv)).astype(np.float32))
    if csr:
        indptr = np.zeros(R + 1, np.int32)
        indptr[1:] = np.cumsum(pages_per)
        table, pind = perm[:indptr[-1]].copy(), indptr
    else:
        width = int(pages_per.max()) + 1
        table = np.full((R, width), -1, np.int32)
        at = 0
        for r in range(R):
            table[r, :pages_per[r]] = perm[at:at + pages_per[r]]
            at += pages_per[r]
        pind = None
    out = oracle.kv_append(k_src, v_src, app, ctx, k_pool, v_pool, table, page_indptr=pind,
                           v_layout=v_layout, k_scale=ks, v_scale=vs)
    return dict(k_src=k_src, v_src=v_src, app=app, ctx=ctx, prior=prior, n=n, table=table,
                pind=pind, k_pool=k_pool, v_pool=v_pool, k_scale=ks, v_scale=vs, ps=ps,
                out=out, v_layout=v_layout)


def pages_of(c, r):
    if c["pind"] is not None:
        return c["table"][c["pind"][r]:c["pind"][r + 1]]
    return c["table"][r]


def as_float(bits, dtype):
    if dtype == FP8:
        return fp8_values()[bits].astype(np.float64)
    if dtype == torch.bfloat16:
        return oracle.bf16_to_float(bits).astype(np.float64)
    if dtype == torch.float16:
        return bits.view(np.float16).astype(np.float64)
    return bits.astype(np.float64)


def readback(c, r, pos, pools=None, scales=True):
    """(K, V) rows [Hkv, d] at token position `pos` of request r, through the
    page table, dequantised."""
    kp, vp, ksc, vsc, _ = c["out"] if pools is None else pools
    ps = c["ps"]
    page = pages_of(c, r)[pos // ps]
    t = pos % ps
    dt = c["k_pool"].dtype
    k = as_float(kp[page, :, t, :], dt)
    v = as_float(vp[page, :, :, t] if c["v_layout"] == "dmajor" else vp[page, :, t, :], dt)
    if dt == FP8 and scales:
        hkv = k.shape[0]
        k = k * ksc[page * hkv:(page + 1) * hkv, None]
        v = v * vsc[page * hkv:(page + 1) * hkv, None]
    return k, v
