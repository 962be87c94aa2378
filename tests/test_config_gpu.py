"""BASELINE configs 4 and 5 as configs: the headline step shapes, two layers deep,
against tgo's CPU path restated (orc_model_step) on identical inputs
(model/batch_test.go:72-200: a batched step reproduces the reference's logits).

* C4: Qwen3-8B widths (hidden 4096, 32/8 heads, MLP 12288, vocab 151936), int4 (the
  symmetric g32-K pack), page 16, driven by bench.py's workload through the library
  Scheduler: 128 decoding sequences with lognormal(1024, 1.0) contexts clipped to
  [16, 8192] plus 2 prefill chunks of 512 -- 130 members, 1152 rows; and the
  decode-dominated step, the 128 decoders alone (128 rows). Both activation precisions.
* C5: Qwen3-32B widths (hidden 5120, 64/8 heads, MLP 25600), int8, 256 decoding
  sequences on one 2048-token shared prefix (suffixes U[32, 1024]) plus one 1024-token
  chunk, prefix-shared attention on and off.

The device pool holds the synthetic context (tgohip_kv_synth); the CPU model gets a copy
of it, so both steps attend to the same keys and values. The scheduler's step is
replayed with its own ports (tgohip_sched_last_step) through tgohip_step and through the
CPU path: rewriting a step's rows with the same values is idempotent.

Budgets: logits within 2e-3 of the row's largest |logit| (BASELINE's bound) for every
member that worked; greedy ids identical wherever the CPU path's top-two margin exceeds
twice the row's largest logit error (a flip inside that is reduction-order noise on a
near tie, the reference's reading of a divergence, internal/conformance/measure.go:56-66);
such rows are printed and may be at most 2% of the decisions. The scheduler's own tokens
equal the replayed step's device argmax exactly.
"""
import ctypes

import numpy as np
import pytest

import bench
import oracle
import tgo_amd

pytestmark = pytest.mark.gpu
LAYERS = 2


def copy_pool(ctx, cpu, layers, kv_heads, positions):
    """The device pool's K and V, every layer, into the CPU model's pool (f16 bits)."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    k, v, npos = ctx.kv_pointers()
    assert npos == positions
    ck, cv = cpu.kv()
    n = layers * positions * kv_heads * 128
    assert ck.size == n
    for dst, src in ((ck, k), (cv, v)):
        assert hip.hipMemcpy(dst.ctypes.data, src, n * 2, 2) == 0  # device to host


def compare(gpu, ids, cpu, extents, what, bound=2e-3):
    """Logits within `bound` (2e-3) of the row max; ids equal outside near ties.
    -> (decisions, [(row, margin, error, row max) of each near tie])."""
    near, n_live, worst = [], 0, 0.0
    for b, n in enumerate(extents):
        if n == 0:
            continue
        n_live += 1
        rowmax = float(np.abs(cpu[b]).max())
        err = float(np.abs(gpu[b] - cpu[b]).max())
        worst = max(worst, err / rowmax)
        assert err <= bound * rowmax, (what, b, err, rowmax)
        want = int(np.argmax(cpu[b]))
        if int(ids[b]) != want:
            top = np.sort(cpu[b].astype(np.float64))[-2:]
            assert top[1] - top[0] <= 2 * err, (what, "greedy differs", b, int(ids[b]), want)
            near.append((b, top[1] - top[0], err, rowmax))
    print("%s: %d decisions, largest |err| / row max %.3g, near ties %s" %
          (what, n_live, worst, near), flush=True)
    return n_live, near


def open_ctx(cfg, form, pool, seed, cascade=0):
    ctx = tgo_amd.Context(0)
    ctx.set_cascade(cascade)
    ctx.config(LAYERS, cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["ffn"],
               cfg["vocab"], cfg["rms_eps"], cfg["rope_theta"], cfg["block"])
    ctx.kv_alloc(pool)
    ctx.synth_weights(seed, form, 0.02)
    return ctx


def cpu_model(cfg, form, pool, seed):
    cpu = oracle.CPUModel(LAYERS, cfg["hidden"], cfg["heads"], cfg["kv_heads"],
                          cfg["head_dim"], cfg["ffn"], cfg["vocab"], cfg["rms_eps"],
                          cfg["rope_theta"], cfg["block"], pool)
    cpu.synth(seed, form, 0.02)
    return cpu


@pytest.mark.timeout(900)
def test_c4_step_matches_the_cpu_path(torch_gpu):
    cfg, form, pool = bench.C4, tgo_amd.FORM_I4_SYM, bench.POOL
    ctx = open_ctx(cfg, form, pool, bench.SEED)
    cpu = None
    try:
        wl = bench.Workload(tgo_amd, ctx, bench.SEED)
        ctx.kv_synth(bench.SEED, 1.0, min(pool, wl.used_positions + 64 * bench.CHUNK))
        cpu = cpu_model(cfg, form, pool, bench.SEED)
        copy_pool(ctx, cpu, LAYERS, cfg["kv_heads"], pool)
        produced, prefill, decodes, _ = wl.sched.step()  # mode 1, the default
        assert (prefill, decodes) == (2 * bench.CHUNK, bench.DECODERS)
        st, pages, maxp = wl.sched.last_step()
        assert len(st["ids"]) == 1152 and len(st["lengths"]) == bench.SLOTS
        want = cpu.step(st, pages, maxp, layers=LAYERS)
        near, decisions = [], 0
        for precision in (1, 0):
            ctx.set_precision(precision)
            logits, ids, _ = ctx.step(st, pages, maxp)
            if precision == 1:
                for slot, tok, done in produced:
                    assert tok == int(ids[slot]), (slot, tok, int(ids[slot]))
            n, nt = compare(logits, ids, want, st["extents"], "C4 precision %d" % precision)
            decisions, near = decisions + n, near + nt
        assert decisions == 2 * 130
        assert len(near) <= 0.02 * decisions, near
    finally:
        if cpu:
            cpu.close()
        ctx.close()


@pytest.mark.timeout(900)
def test_c4_decode_step_matches_the_cpu_path(torch_gpu):
    """The decode-dominated step bench.py reports beside the headline: C4's 128 decoders
    alone (the two requests mid-prefill finished), 128 rows -- 64-row GEMM tiles, the SwiGLU
    gate/up with two k groups per workgroup, 8-way split-K for QKV, O and down, decode-only
    attention -- both precisions."""
    cfg, form, pool = bench.C4, tgo_amd.FORM_I4_SYM, bench.POOL
    ctx = open_ctx(cfg, form, pool, bench.SEED)
    cpu = None
    try:
        wl = bench.Workload(tgo_amd, ctx, bench.SEED)
        ctx.kv_synth(bench.SEED, 1.0, min(pool, wl.used_positions + 64 * bench.CHUNK))
        wl.decode_only()
        cpu = cpu_model(cfg, form, pool, bench.SEED)
        copy_pool(ctx, cpu, LAYERS, cfg["kv_heads"], pool)
        produced, prefill, decodes, _ = wl.sched.step()
        assert (prefill, decodes) == (0, bench.DECODERS)
        st, pages, maxp = wl.sched.last_step()
        assert len(st["ids"]) == bench.DECODERS
        want = cpu.step(st, pages, maxp, layers=LAYERS)
        near, decisions = [], 0
        for precision in (1, 0):
            ctx.set_precision(precision)
            logits, ids, _ = ctx.step(st, pages, maxp)
            if precision == 1:
                for slot, tok, done in produced:
                    assert tok == int(ids[slot]), (slot, tok, int(ids[slot]))
            n, nt = compare(logits, ids, want, st["extents"], "C4 decode precision %d" % precision)
            decisions, near = decisions + n, near + nt
        assert decisions == 2 * bench.DECODERS
        assert len(near) <= 0.02 * decisions, near
    finally:
        if cpu:
            cpu.close()
        ctx.close()


@pytest.mark.timeout(900)
def test_c5_step_matches_the_cpu_path(torch_gpu):
    cfg, form, pool = bench.C5, tgo_amd.FORM_I8, bench.C5_POOL
    ctx = open_ctx(cfg, form, pool, bench.SEED, cascade=2)
    cpu = None
    try:
        wl = bench.SharedPrefixWorkload(tgo_amd, ctx, bench.SEED)
        ctx.kv_synth(bench.SEED, 1.0, min(pool, wl.used_positions + 32 * bench.C5_CHUNK))
        cpu = cpu_model(cfg, form, pool, bench.SEED)
        copy_pool(ctx, cpu, LAYERS, cfg["kv_heads"], pool)
        produced, prefill, decodes, _ = wl.sched.step()
        assert (prefill, decodes) == (bench.C5_CHUNK, bench.C5_DECODERS)
        st, pages, maxp = wl.sched.last_step()
        # every decoding sequence's table begins with the prefix's 128 shared pages
        rows = np.asarray(pages).reshape(len(st["lengths"]), maxp)
        dec = [b for b, n in enumerate(st["extents"]) if n == 1]
        assert len(dec) == 256 and len({tuple(rows[b, :128]) for b in dec}) == 1
        want = cpu.step(st, pages, maxp, layers=LAYERS)
        near, decisions = [], 0
        for cascade in (2, 0):
            ctx.set_cascade(cascade)
            logits, ids, _ = ctx.step(st, pages, maxp)
            if cascade == 2:
                for slot, tok, done in produced:
                    assert tok == int(ids[slot]), (slot, tok, int(ids[slot]))
            n, nt = compare(logits, ids, want, st["extents"], "C5 cascade %d" % cascade)
            decisions, near = decisions + n, near + nt
        assert decisions == 2 * 257
        assert len(near) <= 0.02 * decisions, near
    finally:
        if cpu:
            cpu.close()
        ctx.close()
