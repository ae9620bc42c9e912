"""Synthetic paged decode batches (the measured workloads and test inputs).

A batch is a dict of tensors in the kernels' layout:
    q        [R, Hq, d]                 (bf16 or fp32)
    k_pool   [num_pages, Hkv, page, d]  token rows
    v_pool   [num_pages, Hkv, d, page]  d-major
    block_table [R, max_pages] int32, ctx_lens [R] int32
    k_scale, v_scale [num_pages, Hkv] fp32 (fp8 pools only): the K and V
                columns of one [num_pages, Hkv, 2] pair array
Pages of a request are distinct pages drawn from a random permutation of the
pool, so KV reads are scattered over HBM the way a serving cache is.

Workloads (sizes as the benchmark specifies them):
  llama3_8b_uniform  Hq 32 / Hkv 8 / d 128 / page 16, bf16, 64 requests x 2048
                     tokens, pool 1,048,576 tokens (65,536 pages)
  llama3_8b_hetero   same shape, 256 requests, context ~ lognormal(median 1024,
                     sigma 1.2) clipped to [16, 32768]
  llama3_8b_shed     same shape, 128 requests, context ~ U{1024..8192}, per-task
                     tau ~ U{ceil(ctx/4)..ctx}
  qwen2_7b_fp8       Hq 28 / Hkv 4 / d 128 / page 16, fp8-e4m3fn KV with
                     per-(page, head) scales ~ U(0.01, 0.1), bf16 Q/out,
                     512 requests, context ~ lognormal(median 2048, sigma 1.2)
                     clipped to [16, 16384]
  mha_fp32_small     fp32, 16 requests, 8 heads (MHA), d 64, page 16,
                     context ~ U{64..512}
"""
from __future__ import annotations

import math

import numpy as np
import torch


def lognormal_ctx(n, median, sigma, lo, hi, rng: np.random.Generator) -> np.ndarray:
    x = np.exp(rng.normal(math.log(median), sigma, size=n))
    return np.clip(np.rint(x), lo, hi).astype(np.int32)


def make_batch(ctx_lens, *, num_q_heads, num_kv_heads, head_dim=128, page_size=16,
               kv_dtype=torch.bfloat16, q_dtype=torch.bfloat16, pool_pages=None,
               value_scale=None, seed=0, device="cuda", fp8_scale_range=(0.01, 0.1),
               n_tables=1) -> dict:
    """Random batch. value_scale multiplies N(0,1) Q/K/V (default 1/sqrt(d) for
    bf16, 1 for fp32; fp8 pools hold fp8(N(0,1)) codes times their scales).
    n_tables > 1 builds that many block tables over disjoint pages of the pool
    (so consecutive steps read different HBM)."""
    ctx = np.asarray(ctx_lens, dtype=np.int64)
    R = ctx.size
    npg = (ctx + page_size - 1) // page_size
    need = int(npg.sum())
    pool_pages = max(pool_pages or 0, need * n_tables)
    hkv, d, ps = num_kv_heads, head_dim, page_size
    g = torch.Generator(device=device).manual_seed(seed)
    if value_scale is None:
        value_scale = 1.0 if kv_dtype == torch.float32 else 1.0 / math.sqrt(d)
    fp8 = hasattr(torch, "float8_e4m3fn") and kv_dtype == torch.float8_e4m3fn

    def rnd(shape, dtype, scale):
        x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
        if scale != 1.0:
            x.mul_(scale)
        return x.to(dtype)

    q = rnd((R, num_q_heads, d), q_dtype, value_scale if not fp8 else 1.0 / math.sqrt(d))
    k_pool = rnd((pool_pages, hkv, ps, d), kv_dtype, 1.0 if fp8 else value_scale)
    v_pool = rnd((pool_pages, hkv, d, ps), kv_dtype, 1.0 if fp8 else value_scale)
    k_scale = v_scale = None
    if fp8:
        lo, hi = fp8_scale_range
        k_scale = torch.rand((pool_pages, hkv), generator=g, device=device) * (hi - lo) + lo
        v_scale = torch.rand((pool_pages, hkv), generator=g, device=device) * (hi - lo) + lo
        # stored as (K, V) pairs per (page, kv-head): k_scale / v_scale are
        # the columns of one [pool_pages, hkv, 2] array
        pairs = torch.stack([k_scale, v_scale], -1).contiguous()
        k_scale, v_scale = pairs[..., 0], pairs[..., 1]

    perm = torch.randperm(pool_pages, generator=g, device=device).to(torch.int32).cpu().numpy()
    maxp = max(int(npg.max()) if R else 1, 1)
    tables = []
    for t in range(n_tables):
        bt = np.zeros((R, maxp), dtype=np.int32)
        off = t * need
        for r in range(R):
            bt[r, :npg[r]] = perm[off:off + npg[r]]
            off += npg[r]
        tables.append(torch.from_numpy(bt).to(device))
    return {
        "q": q, "k_pool": k_pool, "v_pool": v_pool,
        "block_table": tables[0], "block_tables": tables,
        "ctx_lens": torch.from_numpy(ctx.astype(np.int32)).to(device),
        "k_scale": k_scale, "v_scale": v_scale, "page_size": ps,
        "kv_bytes": kv_bytes(ctx, hkv, d, kv_dtype),
    }


def kv_bytes(ctx, hkv, d, kv_dtype, tau=None) -> int:
    """Algorithmic KV bytes of one step: sum_r n_r * Hkv * d * 2 * sizeof(kv)
    (+ the fp8 scales of the pages read), n_r = ctx_r or min(ctx_r, tau_r)."""
    ctx = np.asarray(ctx, dtype=np.int64)
    n = ctx if tau is None else np.minimum(ctx, np.where(np.asarray(tau) > 0, tau, ctx))
    eb = torch.tensor([], dtype=kv_dtype).element_size()
    b = int(n.sum()) * hkv * d * 2 * eb
    if eb == 1:
        b += int(((n + 15) // 16).sum()) * hkv * 2 * 4
    return b


def workload(name: str, seed: int = 0, device: str = "cuda", n_tables: int = 1,
             requests: int | None = None) -> dict:
    """One of the named workloads; `requests` shrinks the batch for tests."""
    rng = np.random.default_rng(seed)
    if name == "llama3_8b_uniform":
        R = requests or 64
        b = make_batch(np.full(R, 2048), num_q_heads=32, num_kv_heads=8,
                       pool_pages=65536 if requests is None else None,
                       seed=seed, device=device, n_tables=n_tables)
    elif name == "llama3_8b_hetero":
        R = requests or 256
        ctx = lognormal_ctx(R, 1024, 1.2, 16, 32768, rng)
        b = make_batch(ctx, num_q_heads=32, num_kv_heads=8, seed=seed, device=device,
                       n_tables=n_tables)
        b["urgency"] = rng.uniform(0.0, 1.0, size=R * 8).astype(np.float32)
    elif name == "llama3_8b_shed":
        R = requests or 128
        ctx = rng.integers(1024, 8193, size=R).astype(np.int32)
        b = make_batch(ctx, num_q_heads=32, num_kv_heads=8, seed=seed, device=device,
                       n_tables=n_tables)
        tau_r = np.array([rng.integers(-(-c // 4), c + 1) for c in ctx], dtype=np.int64)
        b["tau"] = np.repeat(tau_r, 8)
        b["urgency"] = rng.uniform(0.0, 1.0, size=R * 8).astype(np.float32)
    elif name == "qwen2_7b_fp8":
        R = requests or 512
        ctx = lognormal_ctx(R, 2048, 1.2, 16, 16384, rng)
        b = make_batch(ctx, num_q_heads=28, num_kv_heads=4, kv_dtype=torch.float8_e4m3fn,
                       seed=seed, device=device, n_tables=n_tables)
    elif name == "mha_fp32_small":
        R = requests or 16
        ctx = rng.integers(64, 513, size=R).astype(np.int32)
        b = make_batch(ctx, num_q_heads=8, num_kv_heads=8, head_dim=64,
                       kv_dtype=torch.float32, q_dtype=torch.float32, seed=seed,
                       device=device, n_tables=n_tables)
    else:
        raise KeyError(name)
    b["name"] = name
    return b
