"""BASELINE config 2 as an op: ragged paged attention over one launch
(tgohip_paged_attention_replay: the launch planned once, its kernels replayed).

    python -m tgo_amd.attn_bench [--iters 50] [--q f16|f32] [--seed 2] [--only decode|prefill]

Config 2: 64 sequences with context lengths uniform in [1, 4096]; 56 decode rows
(one token each) and 8 prefill chunks of min(256, L) tokens; 32 q / 8 kv heads,
head_dim 128, causal; page 16, each sequence's block table a slice of a seeded
permutation of the pool; Q, K, V N(0,1) (K/V f16; Q f16 or f32). The pool holds
the sequences' pages only (about 537 MB of K+V at E[L]).

Algorithmic bytes per launch (HBM-bound): every position a sequence reads, once
(K and V: sum_s L_s * H_kv * d_h * 2 * 2 B), plus q in and the output out
(T * H * d_h * (2 + 2) with f16 q, * (4 + 4) with f32). Flops: 4 * d_h * H per
visible (query, key) pair. Reported: the median launch time of `iters` replays
(HIP events around the replay, divided by iters), GB/s against 8 TB/s, TFLOP/s
against 2.5 PFLOP/s. --only keeps the 56 decode sequences or the 8 prefill chunks alone
(the same pages), to see what each part of the launch costs.
"""
import argparse
import math

import numpy as np
import torch

import tgo_amd

DH = 128


def c2(seed, only=None):
    rng = np.random.default_rng(seed)
    B, H, Hkv, block = 64, 32, 8, 16
    L = rng.integers(1, 4097, size=B)
    ext = np.ones(B, np.int64)
    ext[56:] = np.minimum(256, L[56:])
    need = (L + block - 1) // block
    pool = int(need.sum())
    perm = rng.permutation(pool)
    maxp = int(need.max())
    pages = np.zeros((B, maxp), np.uint32)
    at = 0
    for s in range(B):
        pages[s, :need[s]] = perm[at:at + need[s]]
        at += need[s]
    if only:
        keep = slice(0, 56) if only == "decode" else slice(56, B)
        L, ext, pages = L[keep], ext[keep], pages[keep]
        B = len(L)
    return dict(B=B, H=H, Hkv=Hkv, block=block, L=L, ext=ext, pages=pages, maxp=maxp,
                T=int(ext.sum()), pool=pool)


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--iters", type=int, default=50)
    p.add_argument("--q", default="f16", choices=["f16", "f32"])
    p.add_argument("--seed", type=int, default=2)
    p.add_argument("--only", default=None, choices=["decode", "prefill"])
    args = p.parse_args()
    c = c2(args.seed, args.only)
    H, Hkv, T, block = c["H"], c["Hkv"], c["T"], c["block"]
    positions = c["pool"] * block
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    k = torch.randn(positions, Hkv, DH, device="cuda", generator=g).half()
    v = torch.randn(positions, Hkv, DH, device="cuda", generator=g).half()
    qf16 = args.q == "f16"
    q = torch.randn(T, H, DH, device="cuda", generator=g)
    q = q.half() if qf16 else q
    out = torch.empty(T, H, DH, device="cuda", dtype=torch.float16 if qf16 else torch.float32)
    ctx = tgo_amd.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    dt = tgo_amd.F16 if qf16 else tgo_amd.F32
    scale = 1.0 / math.sqrt(DH)
    args_ = (q, T, H, Hkv, k, v, positions, c["L"], c["ext"], c["pages"].ravel(), c["maxp"],
             block, scale, out)
    ctx.paged_attention_replay(*args_, 3, q_dtype=dt, out_dtype=dt)
    torch.cuda.synchronize()
    times = []
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        ctx.paged_attention_replay(*args_, args.iters, q_dtype=dt, out_dtype=dt)
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / args.iters)
    ms = sorted(times)[2]
    qio = T * H * DH * (4 if qf16 else 8)
    kv = int(c["L"].sum()) * Hkv * DH * 2 * 2
    pairs = sum(int(n) * (int(L) - int(n)) + int(n) * (int(n) + 1) // 2
                for L, n in zip(c["L"], c["ext"]))
    flops = 4.0 * DH * H * pairs
    gbps = (kv + qio) / ms / 1e6
    print("config 2%s: %d sequences (%d rows), sum L = %d, q %s" %
          (" (%s only)" % args.only if args.only else "", c["B"], T, int(c["L"].sum()), args.q))
    print("bytes/launch %.1f MB (K+V %.1f MB, q in + out %.1f MB); flops/launch %.2f GFLOP" %
          ((kv + qio) / 1e6, kv / 1e6, qio / 1e6, flops / 1e9))
    print("launch %.2f us (median of 5 x %d replays): %.0f GB/s = %.3f of 8 TB/s; %.1f TFLOP/s "
          "= %.3f of 2.5 PFLOP/s" % (ms * 1e3, args.iters, gbps, gbps / 8000.0,
                                     flops / ms / 1e9, flops / ms / 1e9 / 2500.0))
    ctx.close()


if __name__ == "__main__":
    main()
