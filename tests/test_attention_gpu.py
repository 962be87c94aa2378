"""Ragged paged attention on the GPU against the float64 oracle.

Mirrors internal/conformance/ragged_test.go (C16, C22, C23) and runs
BASELINE config 2. Tolerance (written here, derived the way tolerance.go
derives budgets, relative to max|v| over the attended rows):
    f16 probabilities into the PV MFMA     2^-11      (StoreF16(1))
    q carried as f16 hi+lo                  2^-21 * (1 + max|score|)
      (an f16 q is exact; its scores are scaled once in f32, inside this term)
    f32 accumulation over d_h and over L    (sqrt(d_h) + sqrt(L)) * 2^-24
    exp2 / division                         8 * 2^-23
The f16 cache rounding is not charged: the oracle reads the same f16 K/V.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle
from oracle import host

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_known_answers.json")))
DH = 128


def budget(b, dh=DH):
    rel = (2.0 ** -11 + 2.0 ** -21 * (1 + b["score"]) +
           (math.sqrt(dh) + math.sqrt(max(b["positions"], 1))) * 2.0 ** -24 + 8 * 2.0 ** -23)
    return rel * max(b["value"], 1e-30)


def pad_heads(x, rows, heads, dh):
    """[rows, heads, dh] -> [rows, heads, 128] zero-padded (the probe's d_h is 4)."""
    out = np.zeros((rows, heads, DH), np.float32)
    out[:, :, :dh] = x.reshape(rows, heads, dh)
    return out


def run(ctx, torch, q, k16, v16, lengths, extents, pages, max_pages, block, scale, H, Hkv,
        out_f16=False, q_f16=False):
    T = q.shape[0]
    dq = torch.from_numpy(np.ascontiguousarray(q, np.float16 if q_f16 else np.float32)).cuda()
    dk = torch.from_numpy(np.ascontiguousarray(k16).view(np.int16)).cuda()
    dv = torch.from_numpy(np.ascontiguousarray(v16).view(np.int16)).cuda()
    cap = k16.shape[0]
    dout = torch.full((T, H, DH), float("nan"), dtype=torch.float16 if out_f16 else torch.float32,
                      device="cuda")
    import tgo_amd
    ctx.paged_attention(dq, T, H, Hkv, dk, dv, cap, lengths, extents, pages, max_pages, block,
                        scale, dout, q_dtype=tgo_amd.F16 if q_f16 else tgo_amd.F32,
                        out_dtype=tgo_amd.F16 if out_f16 else tgo_amd.F32)
    torch.cuda.synchronize()
    return dout.float().cpu().numpy()


def probe_inputs(seqs):
    g = GOLD["ragged_probe"]
    H, Hkv, dh, block, pool = g["qheads"], g["kvheads"], g["headdim"], g["block"], g["pool"]
    T = sum(s["extent"] for s in seqs)
    rows = pool * block
    q = pad_heads(host.spread(T * H * dh, g["spread_seeds"]["q"]), T, H, dh)
    k = pad_heads(host.spread(rows * Hkv * dh, g["spread_seeds"]["k"]), rows, Hkv, dh)
    v = pad_heads(host.spread(rows * Hkv * dh, g["spread_seeds"]["v"]), rows, Hkv, dh)
    k16 = k.astype(np.float16).view(np.uint16)
    v16 = v.astype(np.float16).view(np.uint16)
    lengths = [s["length"] for s in seqs]
    extents = [s["extent"] for s in seqs]
    pages = [p for s in seqs for p in s["pages"]]
    return q, k16, v16, lengths, extents, pages


def test_c16_c22_probe_matches_the_oracle(ctx, torch_gpu):
    """C16 over an f16 cache (C22): ragged_test.go:262, :389."""
    g = GOLD["ragged_probe"]
    q, k16, v16, lengths, extents, pages = probe_inputs(g["seqs"])
    got = run(ctx, torch_gpu, q, k16, v16, lengths, extents, pages, g["max_pages"], g["block"],
              g["scale"], g["qheads"], g["kvheads"])
    want, b = oracle.ragged_attention_f64(q, g["qheads"], g["kvheads"], DH, k16, v16, lengths,
                                          extents, pages, g["max_pages"], g["block"], g["scale"])
    err = np.abs(got - want).max()
    assert err <= budget(b), (err, budget(b), b)
    # the padded dims of the value rows are zero, so the output's are too
    assert np.all(got[:, :, 4:] == 0)


def test_c16_mixed_step_equals_the_separate_steps(ctx, torch_gpu):
    """ragged_test.go:295: bit-exact, sequence by sequence."""
    g = GOLD["ragged_probe"]
    q, k16, v16, lengths, extents, pages = probe_inputs(g["seqs"])
    together = run(ctx, torch_gpu, q, k16, v16, lengths, extents, pages, g["max_pages"],
                   g["block"], g["scale"], g["qheads"], g["kvheads"])
    at = 0
    for s in g["seqs"]:
        if s["extent"] == 0:
            continue
        qs = q[at:at + s["extent"]]
        apart = run(ctx, torch_gpu, qs, k16, v16, [s["length"]], [s["extent"]], s["pages"],
                    g["max_pages"], g["block"], g["scale"], g["qheads"], g["kvheads"])
        assert np.array_equal(apart, together[at:at + s["extent"]])
        at += s["extent"]


def test_c16_the_extents_are_read(ctx, torch_gpu):
    """ragged_test.go:343: the 2/1/1 split moves the output and matches the oracle."""
    g = GOLD["ragged_probe"]
    q, k16, v16, lengths, extents, pages = probe_inputs(g["seqs"])
    base = run(ctx, torch_gpu, q, k16, v16, lengths, extents, pages, g["max_pages"], g["block"],
               g["scale"], g["qheads"], g["kvheads"])
    split = [dict(extent=x["extent"], length=x["length"], pages=s["pages"])
             for x, s in zip(g["split_211"], g["seqs"])]
    _, _, _, l2, e2, p2 = probe_inputs(split)
    moved = run(ctx, torch_gpu, q, k16, v16, l2, e2, p2, g["max_pages"], g["block"], g["scale"],
                g["qheads"], g["kvheads"])
    assert not np.array_equal(moved, base)
    want, b = oracle.ragged_attention_f64(q, g["qheads"], g["kvheads"], DH, k16, v16, l2, e2, p2,
                                          g["max_pages"], g["block"], g["scale"])
    assert np.abs(moved - want).max() <= budget(b)


def test_c23_rows_past_the_extents_are_inert(ctx, torch_gpu):
    """ragged_test.go:461: two unclaimed rows leave every claimed row identical and are zero."""
    g = GOLD["ragged_probe"]
    q, k16, v16, lengths, extents, pages = probe_inputs(g["seqs"])
    claimed = run(ctx, torch_gpu, q, k16, v16, lengths, extents, pages, g["max_pages"],
                  g["block"], g["scale"], g["qheads"], g["kvheads"])
    extra = pad_heads(host.spread(2 * g["qheads"] * g["headdim"], g["spread_seeds"]["pad"]), 2,
                      g["qheads"], g["headdim"])
    padded = run(ctx, torch_gpu, np.concatenate([q, extra]), k16, v16, lengths, extents, pages,
                 g["max_pages"], g["block"], g["scale"], g["qheads"], g["kvheads"])
    assert np.array_equal(padded[:len(q)], claimed)
    assert np.all(padded[len(q):] == 0)


def test_a_permuted_page_table_equals_a_contiguous_cache(ctx, torch_gpu):
    """model/paged_test.go:65: permuting the pool and the table together is bit-exact;
    the negative control (:131) -- the same table over the unpermuted pool -- moves."""
    rng = np.random.default_rng(5)
    H, Hkv, block, L, n = 8, 2, 16, 200, 3
    pool = (L + block - 1) // block
    k = rng.standard_normal((pool * block, Hkv, DH)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((pool * block, Hkv, DH)).astype(np.float16).view(np.uint16)
    q = rng.standard_normal((n, H, DH)).astype(np.float32)
    ident = list(range(pool))
    a = run(ctx, torch_gpu, q, k, v, [L], [n], ident, pool, block, 0.125, H, Hkv)
    perm = rng.permutation(pool)
    kp = np.empty_like(k)
    vp = np.empty_like(v)
    for logical, phys in enumerate(perm):
        kp[phys * block:(phys + 1) * block] = k[logical * block:(logical + 1) * block]
        vp[phys * block:(phys + 1) * block] = v[logical * block:(logical + 1) * block]
    b = run(ctx, torch_gpu, q, kp, vp, [L], [n], list(perm), pool, block, 0.125, H, Hkv)
    assert np.array_equal(a, b)
    c = run(ctx, torch_gpu, q, k, v, [L], [n], list(perm), pool, block, 0.125, H, Hkv)
    assert not np.array_equal(a, c)


def test_decode_equals_prefill_last_row(ctx, torch_gpu):
    """nn/attention_test.go:364 / oracle attention_test.go:153: a decode of the last token
    agrees with the chunk's last row (different work decomposition -> tolerance)."""
    rng = np.random.default_rng(9)
    H, Hkv, block, L = 32, 8, 16, 700
    pool = (L + block - 1) // block
    k = rng.standard_normal((pool * block, Hkv, DH)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((pool * block, Hkv, DH)).astype(np.float16).view(np.uint16)
    q = rng.standard_normal((40, H, DH)).astype(np.float32)
    pages = list(range(pool))
    chunk = run(ctx, torch_gpu, q, k, v, [L], [40], pages, pool, block, 0.088, H, Hkv)
    dec = run(ctx, torch_gpu, q[-1:], k, v, [L], [1], pages, pool, block, 0.088, H, Hkv)
    want, b = oracle.ragged_attention_f64(q[-1:], H, Hkv, DH, k, v, [L], [1], pages, pool, block,
                                          0.088)
    assert np.abs(dec - want).max() <= budget(b)
    assert np.abs(chunk[-1:] - want).max() <= budget(b)


def c2_inputs(seed=2):
    """64 sequences, L ~ U[1,4096], 56 decode + 8 chunks of 256,
    32 q / 8 kv heads, d_h 128, page 16, tables a seeded permutation of the pool."""
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
    T = int(ext.sum())
    k = rng.standard_normal((pool * block, Hkv, DH), dtype=np.float32).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((pool * block, Hkv, DH), dtype=np.float32).astype(np.float16).view(np.uint16)
    q = rng.standard_normal((T, H, DH), dtype=np.float32)
    return dict(B=B, H=H, Hkv=Hkv, block=block, L=L, ext=ext, pages=pages, maxp=maxp, T=T, k=k,
                v=v, q=q, scale=1.0 / math.sqrt(DH))


def test_c2_config_matches_the_oracle_on_every_row(ctx, torch_gpu):
    """BASELINE config 2 in one launch against the float64 oracle: every row of all 64
    sequences (56 decode rows, 8 chunks of up to 256 rows), each sequence within its own
    budget; and the same launch twice is bit-identical."""
    c = c2_inputs()
    got = run(ctx, torch_gpu, c["q"], c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(),
              c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"])
    cu = np.concatenate([[0], np.cumsum(c["ext"])])
    for s in range(c["B"]):
        L, n = int(c["L"][s]), int(c["ext"][s])
        rows = slice(cu[s], cu[s + 1])
        want, b = oracle.ragged_attention_f64(c["q"][rows], c["H"], c["Hkv"], DH, c["k"], c["v"],
                                              [L], [n], c["pages"][s], c["maxp"], c["block"],
                                              c["scale"])
        err = np.abs(got[rows] - want).max()
        assert err <= budget(b), (s, L, n, err, budget(b))
    again = run(ctx, torch_gpu, c["q"], c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(),
                c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"])
    assert np.array_equal(got, again)


def test_c2_mixed_equals_apart_at_full_size(ctx, torch_gpu):
    """Size-independent property at the BASELINE shape: each sequence's rows in the
    64-sequence launch equal the same sequence launched alone, bit for bit."""
    c = c2_inputs(3)
    got = run(ctx, torch_gpu, c["q"], c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(),
              c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"])
    cu = np.concatenate([[0], np.cumsum(c["ext"])])
    for s in (0, 17, 55, 56, 63):
        rows = slice(cu[s], cu[s + 1])
        alone = run(ctx, torch_gpu, c["q"][rows], c["k"], c["v"], [c["L"][s]], [c["ext"][s]],
                    c["pages"][s], c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"])
        assert np.array_equal(alone, got[rows]), s


def test_f16_queries_match_the_oracle(ctx, torch_gpu):
    """An f16 q (the f16-activation mode's) takes one MFMA per product, the scores
    scaled in f32 afterwards: against the oracle fed the same f16 values, on the C16
    probe and on every row of config 2 (decode rows and chunk rows); and mixed
    equals apart, bit for bit."""
    g = GOLD["ragged_probe"]
    q, k16, v16, lengths, extents, pages = probe_inputs(g["seqs"])
    q16 = q.astype(np.float16)
    got = run(ctx, torch_gpu, q16, k16, v16, lengths, extents, pages, g["max_pages"], g["block"],
              g["scale"], g["qheads"], g["kvheads"], q_f16=True)
    want, b = oracle.ragged_attention_f64(q16.astype(np.float32), g["qheads"], g["kvheads"], DH,
                                          k16, v16, lengths, extents, pages, g["max_pages"],
                                          g["block"], g["scale"])
    assert np.abs(got - want).max() <= budget(b)
    c = c2_inputs(5)
    q16 = c["q"].astype(np.float16)
    got = run(ctx, torch_gpu, q16, c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(),
              c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"], q_f16=True)
    cu = np.concatenate([[0], np.cumsum(c["ext"])])
    for s in range(c["B"]):
        L, n = int(c["L"][s]), int(c["ext"][s])
        rows = slice(cu[s], cu[s + 1])
        want, b = oracle.ragged_attention_f64(q16[rows].astype(np.float32), c["H"], c["Hkv"], DH,
                                              c["k"], c["v"], [L], [n], c["pages"][s],
                                              c["maxp"], c["block"], c["scale"])
        err = np.abs(got[rows] - want).max()
        assert err <= budget(b), (s, L, n, err, budget(b))
    for s in (0, 56, 63):
        rows = slice(cu[s], cu[s + 1])
        alone = run(ctx, torch_gpu, q16[rows], c["k"], c["v"], [c["L"][s]], [c["ext"][s]],
                    c["pages"][s], c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"], q_f16=True)
        assert np.array_equal(alone, got[rows]), s


def test_f16_output_is_the_rounded_f32_output(ctx, torch_gpu):
    c = c2_inputs(4)
    f32 = run(ctx, torch_gpu, c["q"], c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(),
              c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"])
    f16 = run(ctx, torch_gpu, c["q"], c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(),
              c["maxp"], c["block"], c["scale"], c["H"], c["Hkv"], out_f16=True)
    assert np.array_equal(f32.astype(np.float16).astype(np.float32), f16)


def test_refusals_name_the_field(ctx, torch_gpu):
    import tgo_amd
    q = np.zeros((1, 4, DH), np.float32)
    k = np.zeros((32, 2, DH), np.uint16)
    with pytest.raises(tgo_amd.TgoError, match="page"):
        # a page beyond the pool
        run(ctx, torch_gpu, q, k, k, [20], [1], [0, 7], 2, 16, 0.5, 4, 2)
    with pytest.raises(tgo_amd.TgoError, match="extents sum"):
        run(ctx, torch_gpu, q, k, k, [5, 5], [1, 1], [0, 0, 1, 1], 2, 16, 0.5, 4, 2)


def shared_prefix_inputs(seed, B, H, Hkv, block, prefix_pages, suffix_lo, suffix_hi, extra=0):
    """B decode sequences whose page tables begin with the same prefix_pages
    pages, each followed by its own pages (suffix lengths U[suffix_lo,
    suffix_hi]), then `extra` unrelated decode sequences."""
    rng = np.random.default_rng(seed)
    P = prefix_pages * block
    L = [P + int(rng.integers(suffix_lo, suffix_hi + 1)) for _ in range(B)]
    L += [int(rng.integers(64, 700)) for _ in range(extra)]
    B2 = B + extra
    need = [(x + block - 1) // block for x in L]
    own = [need[s] - (prefix_pages if s < B else 0) for s in range(B2)]
    pool = prefix_pages + sum(own)
    perm = rng.permutation(pool)
    shared = perm[:prefix_pages]
    at = prefix_pages
    maxp = max(need)
    pages = np.zeros((B2, maxp), np.uint32)
    for s in range(B2):
        row = list(shared) if s < B else []
        row += list(perm[at:at + own[s]])
        at += own[s]
        pages[s, :len(row)] = row
    k = rng.standard_normal((pool * block, Hkv, DH), dtype=np.float32).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((pool * block, Hkv, DH), dtype=np.float32).astype(np.float16).view(np.uint16)
    q = rng.standard_normal((B2, H, DH), dtype=np.float32)
    return dict(L=np.array(L), ext=np.ones(B2, np.int64), pages=pages, maxp=maxp, k=k, v=v, q=q,
                B=B2, H=H, Hkv=Hkv, block=block)


@pytest.mark.parametrize("H,Hkv", [(32, 8), (64, 8)])
def test_shared_prefix_attention_matches_the_oracle(ctx, torch_gpu, H, Hkv):
    """Prefix-shared (cascade) attention: 40 decode sequences over one 512-position
    prefix plus their own suffixes, beside unrelated sequences. Every row equals
    the ragged oracle to tgo's budget and the plain path within f32 rounding;
    the result is the same on a second launch (deterministic)."""
    c = shared_prefix_inputs(21, 40, H, Hkv, 16, 32, 1, 900, extra=5)
    args = (c["q"], c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(), c["maxp"], c["block"],
            1.0 / math.sqrt(DH), H, Hkv)
    plain = run(ctx, torch_gpu, *args)
    ctx.set_cascade(2)
    try:
        shared = run(ctx, torch_gpu, *args)
        again = run(ctx, torch_gpu, *args)
    finally:
        ctx.set_cascade(0)
    assert np.array_equal(shared, again)
    assert not np.array_equal(shared, plain)  # the prefix really took the grouped path
    for s in range(c["B"]):
        want, b = oracle.ragged_attention_f64(c["q"][s:s + 1], H, Hkv, DH, c["k"], c["v"],
                                              [c["L"][s]], [1], c["pages"][s], c["maxp"],
                                              c["block"], 1.0 / math.sqrt(DH))
        assert np.abs(shared[s:s + 1] - want).max() <= budget(b), s
        assert np.abs(shared[s:s + 1] - plain[s:s + 1]).max() <= budget(b), s


def test_shared_prefix_stops_where_the_tables_diverge(ctx, torch_gpu):
    """Members sharing 8 pages with one that diverges after 5: the group's prefix
    is cut to the whole tiles all of them share (4 pages = 64 positions)."""
    c = shared_prefix_inputs(22, 6, 32, 8, 16, 8, 10, 200)
    pages = c["pages"].copy()
    pages[5, 5] = pages[5, 9]  # sequence 5 diverges at page 5
    pages[5, 9] = c["pages"][5, 5]
    args = (c["q"], c["k"], c["v"], c["L"], c["ext"], pages.ravel(), c["maxp"], c["block"],
            1.0 / math.sqrt(DH), 32, 8)
    ctx.set_cascade(2)
    try:
        got = run(ctx, torch_gpu, *args)
    finally:
        ctx.set_cascade(0)
    for s in range(c["B"]):
        want, b = oracle.ragged_attention_f64(c["q"][s:s + 1], 32, 8, DH, c["k"], c["v"],
                                              [c["L"][s]], [1], pages[s], c["maxp"], c["block"],
                                              1.0 / math.sqrt(DH))
        assert np.abs(got[s:s + 1] - want).max() <= budget(b), s


def test_c5_shaped_shared_prefix_every_row(ctx, torch_gpu):
    """BASELINE config 5's attention shape: 256 sequences over one 2048-token prefix
    (128 pages of 16) plus unique suffixes U[32, 1024], 64 q / 8 kv heads. Every row
    against the oracle, and against the plain path."""
    c = shared_prefix_inputs(5, 256, 64, 8, 16, 128, 32, 1024)
    args = (c["q"], c["k"], c["v"], c["L"], c["ext"], c["pages"].ravel(), c["maxp"], c["block"],
            1.0 / math.sqrt(DH), 64, 8)
    plain = run(ctx, torch_gpu, *args)
    ctx.set_cascade(2)
    try:
        shared = run(ctx, torch_gpu, *args)
    finally:
        ctx.set_cascade(0)
    for s in range(256):
        want, b = oracle.ragged_attention_f64(c["q"][s:s + 1], 64, 8, DH, c["k"], c["v"],
                                              [c["L"][s]], [1], c["pages"][s], c["maxp"],
                                              c["block"], 1.0 / math.sqrt(DH))
        assert np.abs(shared[s:s + 1] - want).max() <= budget(b), s
    # both paths round probabilities to f16 for the PV MFMA, against different
    # running maxima: each is within 2^-11 of exact, so they agree to 2^-10
    rel = np.abs(shared - plain).max() / np.abs(plain).max()
    assert rel <= 2.0 ** -10, rel
