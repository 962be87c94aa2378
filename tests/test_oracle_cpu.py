"""The oracle (the CPU restatement of tgo's batched path) pinned against the
reference's own known answers (tests/golden/reference_known_answers.json),
closed forms and exhaustive checks. CPU only."""
import json
import math
import os

import numpy as np
import pytest

import oracle
from oracle import host

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_known_answers.json")))
P = oracle.ptr
L = oracle.lib
TOL = 4 * 2.0 ** -52


def f64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def close(a, b, tol):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.all(np.abs(a - b) <= tol * np.maximum(1.0, np.abs(b)))


# ---- internal/oracle known answers -------------------------------------------

@pytest.mark.parametrize("case", GOLD["rmsnorm"])
def test_rmsnorm_known_answers(case):
    x, g = f64(case["x"]), f64(case["gain"])
    out = np.empty_like(x)
    L.orc_rmsnorm_f64(P(x), P(g), len(x) // len(g), len(g), case["eps"], P(out))
    assert close(out, case["want"], TOL)


def test_rmsnorm_normalizes_each_row_independently():
    # oracle_test.go:89-104: [2,2] with a width-2 gain gives unit rows; one row of 4 does not
    x = f64([1, 1, 100, 100])
    rows = np.empty(4)
    L.orc_rmsnorm_f64(P(x), P(f64([1, 1])), 2, 2, 0.0, P(rows))
    assert close(rows, [1, 1, 1, 1], TOL)
    wide = np.empty(4)
    L.orc_rmsnorm_f64(P(x), P(f64([1, 1, 1, 1])), 1, 4, 0.0, P(wide))
    assert not close(wide[0], 1.0, 1e-3)


@pytest.mark.parametrize("case", GOLD["matmul"])
def test_matmul_known_answers(case):
    out = np.empty(case["m"] * case["n"])
    L.orc_matmul_f64(P(f64(case["x"])), P(f64(case["w"])), case["m"], case["k"], case["n"], P(out))
    assert close(out, case["want"], TOL)


@pytest.mark.parametrize("case", GOLD["silu"])
def test_silu_known_answers(case):
    x = f64(case["x"])
    out = np.empty_like(x)
    L.orc_silu_f64(P(x), len(x), P(out))
    assert close(out, case["want"], TOL)


def test_swiglu_is_silu_times_up():
    g, u = f64([0, 1, -2, 3]), f64([5, -1, 2, 0.5])
    s, out = np.empty(4), np.empty(4)
    L.orc_silu_f64(P(g), 4, P(s))
    L.orc_swiglu_f64(P(g), P(u), 4, P(out))
    assert np.array_equal(out, s * u)


@pytest.mark.parametrize("case", GOLD["softmax"])
def test_softmax_known_answers(case):
    x = f64(case["x"])
    out = np.empty_like(x)
    L.orc_softmax_f64(P(x), len(x), P(out))
    assert close(out, case["want"], TOL)


def test_gather_rows_known_answer():
    c = GOLD["gather_rows"][0]
    ids = np.ascontiguousarray(np.asarray(c["ids"], np.int32))
    out = np.empty(len(c["ids"]) * c["width"])
    L.orc_gather_rows_f64(P(f64(c["table"])), c["vocab"], c["width"], P(ids), len(ids), P(out))
    assert np.array_equal(out, c["want"])


def attention(q, k, v, qseq, qh, kvh, dh, kvlen, scale, base):
    out = np.empty(qseq * qh * dh)
    L.orc_attention_f64(P(f64(q)), P(f64(k)), P(f64(v)), qseq, qh, kvh, dh, kvlen, scale, base,
                        P(out))
    return out


def test_attention_known_answers():
    a, b, c = GOLD["attention"]
    got = attention(a["q"], a["k"], a["v"], 1, 1, 1, 3, 1, a["scale"], a["base"])
    assert np.array_equal(got, a["v"])  # one key: exactly the value
    got = attention(b["q"], b["k"], b["v"], 1, 1, 1, 2, 2, b["scale"], b["base"])
    e0, e1 = math.exp(2.0), math.exp(0.0)
    w0, w1 = e0 / (e0 + e1), e1 / (e0 + e1)
    assert close(got, [w0 * 1 + w1 * 3, w0 * 2 + w1 * 4], 4 * TOL)
    rng = np.random.default_rng(72)
    got = attention(rng.standard_normal(2), rng.standard_normal(8), c["v"], 1, 1, 1, 2, 4, 0.0,
                    c["base"])
    assert close(got, c["want"], 8 * TOL)  # scale 0 averages the values


def test_attention_gqa_grouping_is_floor_division():
    g = GOLD["gqa_grouping"]
    rng = np.random.default_rng(21)
    v = np.zeros((g["kvlen"], g["kvheads"], g["headdim"]))
    for h, val in enumerate(g["v_per_kv_head"]):
        v[:, h, :] = val
    got = attention(rng.standard_normal(4 * 2), rng.standard_normal(2 * 2 * 2), v.ravel(), 1, 4, 2,
                    2, 2, 0.7, 1)
    assert close(got, g["want"], 4 * TOL)


def test_attention_masks_the_future_and_decode_equals_prefill_last_row():
    rng = np.random.default_rng(33)
    q, k, v = rng.standard_normal(3 * 2), rng.standard_normal(3 * 2), rng.standard_normal(3 * 2)
    before = attention(q, k, v, 3, 1, 1, 2, 3, 0.5, 0)
    k2, v2 = k.copy(), v.copy()
    k2[4:] += 5
    v2[4:] += 5
    after = attention(q, k2, v2, 3, 1, 1, 2, 3, 0.5, 0)
    assert np.array_equal(before[:4], after[:4]) and not np.array_equal(before[4:], after[4:])
    dec = attention(q[4:], k, v, 1, 1, 1, 2, 3, 0.5, 2)
    assert np.array_equal(dec, before[4:])


def rope(x, rows, width, rotary, base, pos, style):
    out = np.empty(rows * width)
    p = np.ascontiguousarray(np.asarray(pos, np.int32))
    L.orc_rope_f64(P(f64(x)), rows, width, rotary, base, P(p), style, P(out))
    return out


def test_rope_angle_and_theta_divide_by_rotary_dim():
    g = GOLD["rope_angle"]
    got = rope(g["x"], 1, 4, 4, g["base"], [g["pos"]], 1)
    m = float(g["pos"])
    t1 = g["base"] ** -0.5
    assert close(got, [math.cos(m), math.sin(m), math.cos(m * t1), math.sin(m * t1)], TOL)
    g = GOLD["rope_theta_rotary"]
    got = rope(g["x"], 1, 8, 4, g["base"], [g["pos"]], 1)
    t = g["base"] ** (-2.0 / 4.0)
    assert close(got[2:4], [math.cos(2 * t), math.sin(2 * t)], TOL)
    assert np.array_equal(got[4:], [9, 9, 9, 9])


def test_rope_half_split_is_interleaved_under_the_permutation():
    # rope_test.go:66: permute, rotate interleaved, unpermute == half-split, exactly
    rng = np.random.default_rng(7)
    rows, width = 6, 128
    x = rng.standard_normal(rows * width)
    pos = rng.integers(0, 4096, rows)
    direct = rope(x, rows, width, width, 1e6, pos, 2)
    xp = x.reshape(rows, width)
    perm = np.empty_like(xp)
    perm[:, 0::2], perm[:, 1::2] = xp[:, :64], xp[:, 64:]
    r = rope(perm.ravel(), rows, width, width, 1e6, pos, 1).reshape(rows, width)
    back = np.concatenate([r[:, 0::2], r[:, 1::2]], axis=1)
    assert np.array_equal(direct, back.ravel())
    assert np.array_equal(rope(x, rows, width, width, 1e6, [0] * rows, 1), x)  # position 0


# ---- weights/convert.go ---------------------------------------------------------

def f16(x):
    return int(L.orc_f32_to_f16_bits(float(x), None))


def test_f16_ties_to_even():
    for x, want in GOLD["f16_ties"]["cases"]:
        assert np.uint16(f16(x)).view(np.float16) == np.float16(want), x


def test_f16_saturates_flushes_and_canonical_nan():
    for x, sat in GOLD["f16_saturate"]["cases"]:
        xv = float(x) if not isinstance(x, str) else float(x)
        s = np.zeros(1, np.int32)
        bits = int(L.orc_f32_to_f16_bits(xv, P(s)))
        assert bool(s[0]) == sat, x
        v = float(np.uint16(bits).view(np.float16))
        assert math.isfinite(v) and math.copysign(1, v) == math.copysign(1, xv)
        if sat:
            assert abs(v) == 65504
    for x in GOLD["f16_flush"]["cases"]:
        xv = -0.0 if x == "-0" else float(x)
        bits = f16(xv)
        assert bits & 0x7FFF == 0
        assert bits == (np.float32(xv).view(np.uint32) >> 16) & 0x8000
    assert np.uint16(f16(GOLD["f16_flush"]["smallest_normal"])).view(np.float16) == 2.0 ** -14
    assert f16(float("nan")) == 0x7E00
    c = GOLD["to_f16_counts"]
    src = np.asarray(c["plane"], np.float32)
    out = np.empty(4, np.uint16)
    assert L.orc_to_f16(P(src), P(out), 4) == c["saturated"]


def f32_patterns():
    """Every f32 sign/exponent/top-10-mantissa pattern (2^19) with 16 choices of the low 13
    bits: 0, 1, just under / at / just over the half-way point 0x1000, all ones, and ten
    seeded others -- every rounding boundary of an f16 narrowing, normal or subnormal (the
    round bit of an f16 subnormal lies in the exhaustive upper bits)."""
    low = np.asarray([0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF] +
                     list(np.random.default_rng(9).integers(2, 0x1FFF, 10)), np.uint32)
    high = np.arange(1 << 19, dtype=np.uint32) << np.uint32(13)
    return np.ascontiguousarray((high[:, None] | low[None, :]).ravel())


def test_f16_conversions_over_every_rounding_boundary():
    """The IEEE narrowing equals numpy's float16 cast (NaN by class); the loader rule equals
    it on the normal range and carves out exactly overflow (saturate), f16 subnormals (flush)
    and NaN (canonical) -- convert_test.go:193-232 extended from 2^16 to 2^23 patterns."""
    bits = f32_patterns()
    n = bits.size
    ieee = np.empty(n, np.uint16)
    load = np.empty(n, np.uint16)
    L.orc_f16_ieee_bits_array(P(bits), P(ieee), n)
    L.orc_f16_loader_bits_array(P(bits), P(load), n)
    x = bits.view(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ieee[~nan], ref[~nan])
    assert np.all((ieee[nan] & 0x7C00) == 0x7C00) and np.all((ieee[nan] & 0x3FF) != 0)
    a = np.abs(x)
    normal = (a >= 2.0 ** -14) & (a <= 65504) & ~nan
    assert np.array_equal(load[normal], ref[normal])
    over = (a > 65504) & ~nan
    assert np.all((load[over] & 0x7FFF) == 0x7BFF)
    assert np.array_equal(load[over] >> 15, (bits[over] >> 31).astype(np.uint16))
    sub = a < 2.0 ** -14
    assert np.array_equal(load[sub], ((bits[sub] >> 16) & 0x8000).astype(np.uint16))
    assert np.all(load[nan] == 0x7E00)


def test_transpose_and_permute_heads():
    t = GOLD["transpose"]
    src = np.asarray(t["x"], np.float32)
    dst = np.empty(6, np.float32)
    L.orc_transpose(P(src), P(dst), 2, 3)
    assert np.array_equal(dst, t["want"])
    back = np.empty(6, np.float32)
    L.orc_transpose(P(dst), P(back), 3, 2)
    assert np.array_equal(back, src)
    p = GOLD["permute_heads"]
    x = np.asarray(p["x"], np.float32)
    assert L.orc_permute_heads(P(x), 8, p["last_axis"], p["head_dim"]) == 0
    assert np.array_equal(x, p["want"])
    assert L.orc_permute_heads(P(x), 8, 8, 3) != 0


def test_int8_scale_is_peak_over_127_and_reconstructs_within_half_a_step():
    """weights/weights_test.go:280-288; a windowed quantization equals the whole (convert_test.go:436)."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal(32 * 40 + 7) * 0.3).astype(np.float32)
    q = np.empty(w.size, np.int8)
    s = np.empty((w.size + 31) // 32, np.uint16)
    L.orc_quantize_int8(P(w), w.size, P(q), P(s))
    back = oracle.dequant(1, 1, w.size, q, s).ravel()
    sv = s.view(np.float16).astype(np.float64)
    for b in range(len(s)):
        blk = w[b * 32:(b + 1) * 32]
        assert s[b] == np.float32(np.abs(blk).max() / np.float32(127)).astype(np.float16).view(np.uint16)
        assert np.all(np.abs(back[b * 32:(b + 1) * 32] - blk) <= sv[b] / 2 + 1e-7)
    q2, s2 = np.empty(64, np.int8), np.empty(2, np.uint16)
    L.orc_quantize_int8(P(w[32:96].copy()), 64, P(q2), P(s2))
    assert np.array_equal(q2, q[32:96]) and np.array_equal(s2, s[1:3])


def test_int4_tgo_layout_and_bound():
    """The int4 triple: 8 codes per word low nibble first, f16 scale and integer zero per
    128 flattened elements; the matmul error is inside tgo's (1/30) sum|x| range bound
    (tolerance.go:151-175, reaudit_test.go:249-300). Bit layout: parity unpinned (accel's
    quantizer is absent); pinned here by closed form."""
    rng = np.random.default_rng(2)
    k, n = 256, 5 * 64
    w = (rng.standard_normal(k * n) * 0.05).astype(np.float32)
    c = np.empty((k * n + 7) // 8, np.uint32)
    s = np.empty((k * n + 127) // 128, np.uint16)
    z = np.empty_like(s)
    L.orc_quantize_int4_tgo(P(w), w.size, P(c), P(s), P(z))
    back = oracle.dequant(2, k, n, c, s, z).ravel()
    nib = (c[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    zv = z.view(np.float16).astype(np.float32)
    assert np.all(zv == np.round(zv)) and np.all((zv >= 0) & (zv <= 15))
    want = (nib.ravel()[:k * n].astype(np.float32) - np.repeat(zv, 128)[:k * n]) * \
        np.repeat(s.view(np.float16).astype(np.float32), 128)[:k * n]
    assert np.array_equal(back, want)
    x = rng.standard_normal(k).astype(np.float32)
    exact = x.astype(np.float64) @ w.reshape(k, n).astype(np.float64)
    got = x.astype(np.float64) @ back.reshape(k, n).astype(np.float64)
    for col in range(0, n, 37):
        bound = L.orc_int4_tgo_bound(P(x), P(s), P(z), k, n, col)
        assert abs(got[col] - exact[col]) <= bound + 1e-12


def test_int4_tgo_quantizer_follows_the_range_over_fifteen_rule():
    """What the mathematics fixes about the int4 triple (tolerance.go:150-160: "a group's
    range over fifteen"): per group of 128 flattened elements the stored scale is
    f16((max - min) / 15) (so a step of range/16 fails), the zero is round(-min / s)
    clamped to [0, 15], and each code is round(x / s + z) clamped to [0, 15], so every
    element not at a clamp reconstructs within half a step. Ties round to even (this
    build's rule; accel's quantizer is absent and its bit layout parity unpinned)."""
    rng = np.random.default_rng(9)
    n = 128 * 24 + 40  # a ragged last group
    w = (rng.standard_normal(n) * 0.05).astype(np.float32)
    w[128:256] += 0.04   # all-positive-ish group: the zero clamps low
    w[256:384] = 0.125   # a flat group
    c = np.empty((n + 7) // 8, np.uint32)
    s = np.empty((n + 127) // 128, np.uint16)
    z = np.empty_like(s)
    L.orc_quantize_int4_tgo(P(w), n, P(c), P(s), P(z))
    q = ((c[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).ravel()[:n]
    for g in range(len(s)):
        blk = w[g * 128:(g + 1) * 128]
        mn, mx = np.float32(blk.min()), np.float32(blk.max())
        step = np.float32((mx - mn) / np.float32(15))
        want_s = oracle.f16_bits(np.float32(step if step > 0 else 1.0))
        assert s[g] == want_s, g
        assert s[g] != oracle.f16_bits(np.float32((mx - mn) / np.float32(16))) or step == 0
        sv = float(np.float16(s.view(np.float16)[g]))
        zv = float(np.float16(z.view(np.float16)[g]))
        assert zv == min(15.0, max(0.0, float(np.round(-float(mn) / sv))))
        want_q = np.clip(np.round(blk.astype(np.float64) / sv + zv), 0, 15)
        assert np.array_equal(q[g * 128:(g + 1) * 128], want_q.astype(np.uint32)), g
        back = (want_q - zv) * sv
        inside = (want_q > 0) & (want_q < 15)
        assert np.all(np.abs(back - blk)[inside] <= sv / 2 * (1 + 1e-6)), g
    assert float(np.float16(s.view(np.float16)[2])) == 1.0  # flat group: step 1


def test_int8_rounds_half_steps_to_even():
    """The int8 rule on a constructed block: peak 127 gives the exact scale 1.0, so x/s
    lands on half steps exactly; ties go to even (this build's rule, accel's being
    invisible), and the codes saturate at +-127."""
    w = np.zeros(32, np.float32)
    w[:8] = [127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5]
    q = np.empty(32, np.int8)
    s = np.empty(1, np.uint16)
    L.orc_quantize_int8(P(w), 32, P(q), P(s))
    assert float(s.view(np.float16)[0]) == 1.0
    assert q[:8].tolist() == [127, 2, 4, -2, -4, 0, 0, 126]


def test_int4_sym_closed_form():
    """The BASELINE pack on a tiny hand-built plane: w[k][n] = (nibble - 8) * s[k/32][n]."""
    K, N = 64, 2
    nibbles = np.arange(K * N).reshape(K, N) % 16
    qw = np.zeros((K // 8, N), np.uint32)
    for kk in range(K):
        for nn in range(N):
            qw[kk // 8, nn] |= np.uint32(nibbles[kk, nn]) << np.uint32(4 * (kk % 8))
    sc = np.asarray([[1.0, 0.5], [0.25, 2.0]], np.float16).view(np.uint16)
    got = oracle.dequant(3, K, N, qw, sc)
    want = (nibbles - 8) * np.repeat(sc.view(np.float16).astype(np.float32), 32, axis=0)
    assert np.array_equal(got, want)


def test_synth_generator_is_the_documented_one():
    """orc_normal: Irwin-Hall of twelve 21-bit uniforms minus six, from splitmix64."""
    def sm(x):
        x = (x + 0x9E3779B97F4A7C15) & (2 ** 64 - 1)
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & (2 ** 64 - 1)
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & (2 ** 64 - 1)
        return x ^ (x >> 31)
    def h3(seed, stream, idx):
        return sm((sm((seed * 0x100000001B3 + stream) & (2 ** 64 - 1)) + idx) & (2 ** 64 - 1))
    for idx in (0, 1, 12345):
        s = 0
        for j in range(4):
            h = h3(7, 3, idx * 4 + j)
            s += (h & 0x1FFFFF) + ((h >> 21) & 0x1FFFFF) + ((h >> 42) & 0x1FFFFF)
        assert L.orc_normal(7, 3, idx) == (s - 6 * 2 ** 21) / 2 ** 21
    v = oracle.synth_normal_f32(1, 2, 200000, 1.0)
    assert abs(v.mean()) < 0.02 and abs(v.std() - 1) < 0.02


# ---- the ragged oracle and the f32 CPU path -----------------------------------

def test_ragged_oracle_reduces_to_dense_attention():
    """One contiguous sequence through the page table equals oracle.Attention."""
    rng = np.random.default_rng(3)
    H, Hkv, dh, Lq, Lk, block = 4, 2, 8, 3, 10, 4
    q = rng.standard_normal((Lq, H, dh)).astype(np.float32)
    k = rng.standard_normal((12, Hkv, dh)).astype(np.float32)
    v = rng.standard_normal((12, Hkv, dh)).astype(np.float32)
    got, _ = oracle.ragged_attention_f64(q, H, Hkv, dh, k, v, [Lk], [Lq], [0, 1, 2], 3, block,
                                         0.35, f16_cache=False)
    want = attention(q.ravel(), k.ravel(), v.ravel(), Lq, H, Hkv, dh, Lk, 0.35, Lk - Lq)
    assert close(got.ravel(), want, 16 * TOL)


def test_ragged_oracle_walks_the_page_table():
    """The C16 probe (ragged_test.go:65-73): permuting the pool with the table changes nothing;
    the same table over the unpermuted pool does."""
    g = GOLD["ragged_probe"]
    H, Hkv, dh, block = g["qheads"], g["kvheads"], g["headdim"], g["block"]
    T = sum(s["extent"] for s in g["seqs"])
    rows = g["pool"] * block
    q = host.spread(T * H * dh, 7).reshape(T, H, dh)
    k = host.spread(rows * Hkv * dh, 13).reshape(rows, Hkv, dh)
    v = host.spread(rows * Hkv * dh, 29).reshape(rows, Hkv, dh)
    lengths = [s["length"] for s in g["seqs"]]
    extents = [s["extent"] for s in g["seqs"]]
    pages = [p for s in g["seqs"] for p in s["pages"]]
    base, b = oracle.ragged_attention_f64(q, H, Hkv, dh, k, v, lengths, extents, pages,
                                          g["max_pages"], block, g["scale"], f16_cache=False)
    perm = np.random.default_rng(0).permutation(g["pool"])
    kp, vp = np.empty_like(k), np.empty_like(v)
    for old, new in enumerate(perm):
        kp[new * block:(new + 1) * block] = k[old * block:(old + 1) * block]
        vp[new * block:(new + 1) * block] = v[old * block:(old + 1) * block]
    pages2 = [int(perm[p]) for p in pages]
    moved, _ = oracle.ragged_attention_f64(q, H, Hkv, dh, kp, vp, lengths, extents, pages2,
                                           g["max_pages"], block, g["scale"], f16_cache=False)
    assert np.array_equal(base, moved)
    wrong, _ = oracle.ragged_attention_f64(q, H, Hkv, dh, k, v, lengths, extents, pages2,
                                           g["max_pages"], block, g["scale"], f16_cache=False)
    assert not np.array_equal(base, wrong)
    assert b["positions"] == 5


NORM_BEFORE_ROPE, NORM_AFTER_ROPE = 0, 1  # qkOrder (model/graph_rig_test.go:286-293)


def reference_forward(cfg, W, ids, f16_cache, order=NORM_BEFORE_ROPE):
    """model/graph_rig_test.go:308-371 restated: float64 forward of a prefill from an empty
    cache, composed of the float64 oracle functions, last row's logits. Every norm takes
    its gain from W. With f16_cache the keys (after norm and RoPE) and values are rounded to
    f16 as a paged f16 pool stores them. order selects q/k-norm before RoPE (Qwen3) or the
    ordering mistake, after it (graph_rig_test.go:335-347)."""
    t, d, H, Hkv, dh, f, V = len(ids), cfg["d"], cfg["H"], cfg["Hkv"], 128, cfg["f"], cfg["V"]
    eps, base = cfg["eps"], cfg["theta"]

    def mm(x, w, m, k, n):
        out = np.empty(m * n)
        L.orc_matmul_f64(P(f64(x)), P(f64(w)), m, k, n, P(out))
        return out

    def rms(x, g, rows, w):
        out = np.empty(rows * w)
        L.orc_rmsnorm_f64(P(f64(x)), P(f64(g)), rows, w, eps, P(out))
        return out

    posq = [p for p in range(t) for _ in range(H)]
    posk = [p for p in range(t) for _ in range(Hkv)]
    h = f64(W["embed"][ids].ravel())
    for l in range(cfg["L"]):
        g = lambda name: W["%d.%s" % (l, name)]
        n = rms(h, g("attn_norm"), t, d)
        q = mm(n, g("wq"), t, d, H * dh)
        k = mm(n, g("wk"), t, d, Hkv * dh)
        v = mm(n, g("wv"), t, d, Hkv * dh)
        if order == NORM_BEFORE_ROPE:
            q = rope(rms(q, g("qnorm"), t * H, dh), t * H, dh, dh, base, posq, 1)
            k = rope(rms(k, g("knorm"), t * Hkv, dh), t * Hkv, dh, dh, base, posk, 1)
        else:
            q = rms(rope(q, t * H, dh, dh, base, posq, 1), g("qnorm"), t * H, dh)
            k = rms(rope(k, t * Hkv, dh, dh, base, posk, 1), g("knorm"), t * Hkv, dh)
        if f16_cache:
            k = k.astype(np.float16).astype(np.float64)
            v = v.astype(np.float16).astype(np.float64)
        a = attention(q, k, v, t, H, Hkv, dh, t, 1 / math.sqrt(dh), 0)
        h = h + mm(a, g("wo"), t, H * dh, d)
        n2 = rms(h, g("ffn_norm"), t, d)
        gt = mm(n2, g("wgate"), t, d, f)
        up = mm(n2, g("wup"), t, d, f)
        act = np.empty(t * f)
        L.orc_swiglu_f64(P(gt), P(up), t * f, P(act))
        h = h + mm(act, g("wdown"), t, f, d)
    last = rms(h[(t - 1) * d:], W["final_norm"], 1, d)
    return mm(last, W["lm_head"], 1, d, V)


def test_cpu_step_matches_the_float64_reference_forward():
    """orc_model_step (tgo's f32 CPU path over an f16 paged pool) against referenceForward,
    to prefillTol (graph_rig_test.go:528-552): 8 * 10 * sqrt(d) * 2^-24 * (2L + 1) on the
    relative deviation |got - want| / (1 + |want|) (graph_rig_test.go:388-398).

    Every norm gain is a distinct f16exact plane (graph_rig_test.go:42-84: multiples of
    1/8 in [-2, 2), negatives and zeros included), so a gain dropped, shared wrongly or
    applied at the wrong place moves the result. Two negative controls show the budget
    tells things apart: the reference with q/k-norm after RoPE (the ordering mistake,
    graph_rig_test.go:286-351) and the reference without the pool's f16 rounding of K and
    V both exceed it."""
    cfg = dict(L=2, d=64, H=4, Hkv=2, f=128, V=96, eps=1e-6, theta=1e6)
    rng = np.random.default_rng(5)
    dh = 128

    def plane(K, N):  # multiples of 1/64 in [-1/4, 1/4): exact in f16
        return (rng.integers(-16, 16, K * N) / 64.0).astype(np.float32).reshape(K, N)

    ports = []  # f16exact gains, one distinct plane per port (graph_rig_test.go:57-84)

    def gain(name, n):
        ports.append(name)
        return np.array([host.f16exact(len(ports) * 7919 + i * 104729 + 1) for i in range(n)],
                        np.float32)

    W = {"embed": plane(cfg["V"], cfg["d"]), "lm_head": plane(cfg["d"], cfg["V"])}
    for l in range(cfg["L"]):
        W["%d.attn_norm" % l] = gain("%d.attn_norm" % l, cfg["d"])
        W["%d.wq" % l] = plane(cfg["d"], cfg["H"] * dh)
        W["%d.wk" % l] = plane(cfg["d"], cfg["Hkv"] * dh)
        W["%d.wv" % l] = plane(cfg["d"], cfg["Hkv"] * dh)
        W["%d.wo" % l] = plane(cfg["H"] * dh, cfg["d"])
        W["%d.qnorm" % l] = gain("%d.qnorm" % l, dh)
        W["%d.knorm" % l] = gain("%d.knorm" % l, dh)
        W["%d.ffn_norm" % l] = gain("%d.ffn_norm" % l, cfg["d"])
        W["%d.wgate" % l] = plane(cfg["d"], cfg["f"])
        W["%d.wup" % l] = plane(cfg["d"], cfg["f"])
        W["%d.wdown" % l] = plane(cfg["f"], cfg["d"])
    W["final_norm"] = gain("final_norm", cfg["d"])
    gains = [n for n in W if n.endswith("norm")]
    assert len(gains) == 4 * cfg["L"] + 1
    allg = np.concatenate([W[n] for n in gains])
    assert (allg < 0).any() and (allg == 0).any() and len(np.unique(allg)) > 20
    assert not np.array_equal(W["0.qnorm"], W["0.knorm"])
    m = oracle.CPUModel(cfg["L"], cfg["d"], cfg["H"], cfg["Hkv"], dh, cfg["f"], cfg["V"],
                        cfg["eps"], cfg["theta"], 4, 64)
    try:
        for name, w in W.items():
            if name in gains:
                m.gain(name, w)
            else:
                m.weight(name, 0, w.shape[0], w.shape[1], oracle.f16_bits(w))
        ids = [3, 17, 40, 8, 95, 0]
        st = host.new_batch_step(cfg["V"], cfg["H"], cfg["Hkv"], len(ids),
                                 [host.Member(ids, 0, [0, 1]), host.Member([], 0, [2])], 4, 64)
        pages = host.page_table([[0, 1], [2]], 16)
        got = m.step(st, pages, 16)[0]
    finally:
        m.close()
    tol = 8 * 10 * math.sqrt(cfg["d"]) * 2.0 ** -24 * (2 * cfg["L"] + 1)
    worst = lambda want: np.max(np.abs(got - want) / (1 + np.abs(want)))
    want = reference_forward(cfg, W, np.asarray(ids), True)
    assert worst(want) <= tol
    assert int(np.argmax(got)) == int(np.argmax(want))
    assert worst(reference_forward(cfg, W, np.asarray(ids), True, NORM_AFTER_ROPE)) > 10 * tol
    assert worst(reference_forward(cfg, W, np.asarray(ids), False)) > tol


def small_step(cfg):
    """A prefill chunk of 7 beside a 3-token member and an idle slot, over scattered pages."""
    rng = np.random.default_rng(12)
    p0 = [int(t) for t in rng.integers(0, cfg["V"], 7)]
    p1 = [int(t) for t in rng.integers(0, cfg["V"], 3)]
    members = [host.Member(p0, 0, [5, 1]), host.Member([], 0, []), host.Member(p1, 0, [9])]
    st = host.new_batch_step(cfg["V"], cfg["H"], cfg["Hkv"], 10, members, 4, 64)
    return st, host.page_table([m.pages for m in members], 4)


@pytest.mark.parametrize("fault", [oracle.FAULT_QKNORM_AFTER_ROPE, oracle.FAULT_QK_UNIT_GAIN,
                                   oracle.FAULT_K_TAKES_Q_GAIN, oracle.FAULT_QK_GAIN_AFTER_ROPE,
                                   oracle.FAULT_NORM_UNIT_GAIN, oracle.FAULT_FINAL_UNIT_GAIN])
@pytest.mark.parametrize("form", [oracle.FORM_F16, oracle.FORM_I4_SYM])
def test_planted_mistakes_move_the_logits_past_the_gpu_bound(form, fault):
    """The GPU step tests hold the device to |gpu - cpu| <= 2e-3 * max|cpu| per row over
    synthesized models. Planted in the CPU path, each plausible kernel mistake around the
    norms -- q/k-norm after RoPE, a q/k gain dropped, k normalized with q's gain, the gain
    applied after the rotation, the attn/ffn gain dropped, the final gain dropped -- moves
    some row by more than ten times that bound, so none of them could pass those tests."""
    cfg = dict(L=2, d=256, H=4, Hkv=2, f=512, V=1024, eps=1e-6, theta=1e6)
    st, pages = small_step(cfg)
    out = {}
    for fl in (oracle.FAULT_NONE, fault):
        m = oracle.CPUModel(cfg["L"], cfg["d"], cfg["H"], cfg["Hkv"], 128, cfg["f"], cfg["V"],
                            cfg["eps"], cfg["theta"], 4, 64)
        try:
            m.synth(11, form, 0.02)
            m.set_fault(fl)
            out[fl] = m.step(st, pages, 4)
        finally:
            m.close()
    good, bad = out[oracle.FAULT_NONE], out[fault]
    assert np.all(good[1] == 0) and np.all(bad[1] == 0)
    moved = max(np.abs(bad[r] - good[r]).max() / np.abs(good[r]).max() for r in (0, 2))
    assert moved > 10 * 2e-3, moved


def test_synthesized_gains_are_f16exact_valued():
    """The synthesizer's gains (shared definition with the device): multiples of 1/8 in
    [-2, 2) -- the value set of f16exact (graph_rig_test.go:42-48) -- with negatives and
    zeros, distinct per port (stream)."""
    a = oracle.synth_gain(3, 2, 4096)  # final_norm's stream
    b = oracle.synth_gain(3, 1 * 64 + 5, 4096)  # layer 0's qnorm
    for g in (a, b):
        assert np.all(g * 8 == np.round(g * 8)) and g.min() == -2 and g.max() == 1.875
        assert (g == 0).any() and (g < 0).mean() > 0.4
        assert oracle.f16_to_f32(oracle.f16_bits(g)).tolist() == g.tolist()
    assert not np.array_equal(a, b)
    want = [((int(L.orc_hash3(3, 2 * 4, i)) % 32) - 16) / 8 for i in range(64)]
    assert a[:64].tolist() == want


def test_top_two_margin_and_argmax_known_answers():
    """TopTwoMargin (measure_test.go:41-76) and argmax's tie rule (stages_test.go:375)."""
    for c in GOLD["top_two_margin"]["cases"]:
        assert abs(host.top_two_margin(np.asarray(c["logits"], np.float32)) - c["want"]) <= 1e-6
    with pytest.raises(host.Refused, match=GOLD["top_two_margin"]["refuses_one_logit"]):
        host.top_two_margin([1.0])
    assert host.argmax_first(GOLD["argmax_ties"]["logits"]) == GOLD["argmax_ties"]["want"]
    nan, inf = float("nan"), float("inf")
    # Go's loops by hand: a NaN is never taken after index 0 (argmax) or 1 (margin)
    assert host.argmax_first([nan, 3, 9]) == 0 and host.argmax_first([1, nan, 9, 9]) == 2
    assert host.argmax_first([-inf, -inf]) == 0
    assert math.isnan(host.top_two_margin([nan, 1, 2]))
    assert math.isnan(host.top_two_margin([5, nan, 3, 4]))  # nothing after displaces x[0]
    assert host.top_two_margin([5, nan, 3, 6]) == 1.0
    assert host.top_two_margin([4, 1, nan, 3]) == 1.0
    assert math.isnan(host.top_two_margin([inf, inf, 1]))
    assert host.top_two_margin([inf, 3]) == inf
