"""Whole batched steps on the GPU against tgo's CPU path restated (oracle.c).

The step is driven like Batch.step (batch.go:314-458): every slot is a
member, the packing is model.NewBatchStep's (restated in oracle/host.py),
pages come from a prefix pool, and the same ports go to the GPU
(tgohip_step) and to the CPU restatement (orc_model_step).

Budgets, written here:
  * logits: |gpu - cpu| <= 2e-3 * max|cpu| per row (BASELINE's 2e-3 relative
    bound, scaled by the row's magnitude);
  * greedy ids (first strict maximum, sample/stages.go:196-206) identical
    for every step, the C1 config's 64-step requirement; the ids are the
    device argmax kernel's, which also equal the Go rule applied to the GPU's
    own logits, exactly, on every step;
  * the device top-two margin (TopTwoMargin, internal/conformance/measure.go:91)
    equals the Go loop over the GPU's logits exactly (float64);
  * batched vs apart (batch_test.go:72-200): 1e-5 relative + same argmax.

The synthesized models carry seeded gains (multiples of 1/8 in [-2, 2),
negatives and zeros included, a distinct plane per port): a kernel that drops a
gain, shares it wrongly across heads or applies q/k-norm after RoPE moves the
logits far past the bound (tests/test_oracle_cpu.py plants each mistake in the
CPU path and measures it). C1 runs with the unit gains its config states and
again with seeded gains.
"""
import numpy as np
import pytest

import oracle
from oracle import host

pytestmark = pytest.mark.gpu


class Engine:
    """Batch.step's host half over a backend that runs the forward pass."""

    def __init__(self, backend, vocab, heads, kv_heads, positions, block, nslots):
        self.backend = backend
        self.V, self.H, self.Hkv, self.block = vocab, heads, kv_heads, block
        self.capacity = positions
        self.max_pages = positions // block
        self.pool = host.Pool(block, positions // block)
        self.slots = [dict(lease=None, length=0) for _ in range(nslots)]

    def admit(self, slot, prompt, reserve):
        lease = self.pool.acquire(prompt, reserve=reserve)
        self.slots[slot] = dict(lease=lease, length=lease.reused)

    def step(self, work):
        members = [host.Member([], s["length"], list(s["lease"].blocks) if s["lease"] else [])
                   for s in self.slots]
        for slot, toks in work:
            s = self.slots[slot]
            need = s["length"] + len(toks)
            if need > len(s["lease"].ids):
                s["lease"].grow(need - len(s["lease"].ids))
            members[slot] = host.Member(list(toks), s["length"], list(s["lease"].blocks))
        rows = sum(len(t) for _, t in work)
        st = host.new_batch_step(self.V, self.H, self.Hkv, rows, members, self.block,
                                 self.capacity)
        table = host.page_table([m.pages for m in members], self.max_pages)
        logits = self.backend(st, table, self.max_pages)
        for slot, toks in work:
            s = self.slots[slot]
            need = s["length"] + len(toks)
            if need > len(s["lease"].ids):
                extra = need - len(s["lease"].ids)
                s["lease"].commit(list(toks[len(toks) - extra:]))
            s["lease"].publish(s["length"] + len(toks))
            s["length"] += len(toks)
        return logits


def go_argmax(row):
    """sample/stages.go:196-206 over a float32 row (numpy's first maximal index is the
    Go rule when the row holds no NaN; the loop otherwise)."""
    if np.isnan(row).any():
        return host.argmax_first(row)
    return int(np.argmax(row))


def go_margin(row):
    """TopTwoMargin (measure.go:91-110): for a row without NaN, the top two of the
    multiset in float64 (a repeated maximum gives 0); the Go loop otherwise."""
    if np.isnan(row).any():
        return host.top_two_margin(row)
    top = np.partition(row, len(row) - 2)[-2:].astype(np.float64)
    return float(top.max() - top.min())


def gpu_backend(ctx, record=None):
    """The device step. Checks, on every step, that the device argmax and top-two
    margin of each member that worked are the Go rules over the GPU's own logits;
    record (a list) collects the device ids."""
    def run(st, table, max_pages):
        logits, ids, _ = ctx.step(st, table, max_pages, want_argmax=True)
        margins = ctx.step_margins(len(st["lengths"]))
        for b, n in enumerate(st["extents"]):
            if n == 0:
                assert ids[b] == -1
                continue
            assert int(ids[b]) == go_argmax(logits[b]), ("device argmax", b)
            assert margins[b] == go_margin(logits[b]), ("device margin", b)
        if record is not None:
            record.append(ids.copy())
        return logits
    return run


def cpu_backend(model):
    def run(st, table, max_pages):
        return model.step(st, table, max_pages)
    return run


def argmax_first(row):
    return go_argmax(row)


def check_logits(gpu, cpu, rows, what):
    for r in rows:
        bound = 2e-3 * np.abs(cpu[r]).max()
        err = np.abs(gpu[r] - cpu[r]).max()
        assert err <= bound, (what, r, err, bound)


SMALL = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1024,
             eps=1e-6, theta=1e6, block=4, positions=256)


def unit_gains(ctx, cpu, cfg):
    """Binds 1.0 to every norm gain on both sides (C1's stated gains)."""
    ports = [("final_norm", cfg["hidden"])]
    for l in range(cfg["layers"]):
        ports += [("%d.attn_norm" % l, cfg["hidden"]), ("%d.ffn_norm" % l, cfg["hidden"]),
                  ("%d.qnorm" % l, 128), ("%d.knorm" % l, 128)]
    for name, w in ports:
        ctx.gain(name, np.ones(w, np.float32))
        cpu.gain(name, np.ones(w, np.float32))


def make_pair(torch, cfg, form, seed, precision):
    import tgo_amd
    ctx = tgo_amd.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    ctx.set_precision(precision)
    ctx.config(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
               cfg["ffn"], cfg["vocab"], cfg["eps"], cfg["theta"], cfg["block"])
    ctx.synth_weights(seed, form, 0.02)
    ctx.kv_alloc(cfg["positions"])
    cpu = oracle.CPUModel(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["kv_heads"],
                          cfg["head_dim"], cfg["ffn"], cfg["vocab"], cfg["eps"], cfg["theta"],
                          cfg["block"], cfg["positions"])
    cpu.synth(seed, form, 0.02)
    return ctx, cpu


@pytest.mark.parametrize("form", [0, 1, 2, 3])
@pytest.mark.parametrize("precision", [0, 1])
def test_mixed_step_matches_the_cpu_path(torch_gpu, form, precision):
    """batch_test.go:72-200's shape: a chunk of 3, a decode, an empty slot, scattered pages."""
    cfg = SMALL
    ctx, cpu = make_pair(torch_gpu, cfg, form, 11 + form, precision)
    try:
        engines = [Engine(b, cfg["vocab"], cfg["heads"], cfg["kv_heads"], cfg["positions"],
                          cfg["block"], 3) for b in (gpu_backend(ctx), cpu_backend(cpu))]
        rng = np.random.default_rng(form)
        p0 = [int(t) for t in rng.integers(0, cfg["vocab"], 7)]
        p1 = [int(t) for t in rng.integers(0, cfg["vocab"], 5)]
        for e in engines:
            e.admit(0, p0, 4)
            e.admit(1, p1, 4)
        # prefill both, then the mixed step: a chunk of 3 for a new slot plus one decode
        outs = [e.step([(0, p0), (1, p1)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1], "prefill")
        p2 = [int(t) for t in rng.integers(0, cfg["vocab"], 3)]
        for e in engines:
            e.admit(2, p2, 4)
        t0 = argmax_first(outs[1][0])
        outs = [e.step([(0, [t0]), (2, p2)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 2], "mixed")
        assert np.all(outs[0][1] == 0)  # the slot with nothing to say
    finally:
        ctx.close()
        cpu.close()


WIDE = dict(layers=1, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=1024,
            eps=1e-6, theta=1e6, block=16, positions=512)


@pytest.mark.parametrize("form", [0, 1, 2, 3])
def test_small_batch_step_on_the_small_m_kernel(torch_gpu, form):
    """Qwen3-8B-wide projections (K = 4096 and 12288) at 3 and 2 rows: the
    small-M kernel runs the QKV (f32 out), O (residual add), gate/up (SwiGLU)
    and LM-head projections, every form, against the CPU path."""
    cfg = WIDE
    ctx, cpu = make_pair(torch_gpu, cfg, form, 31 + form, 0)
    try:
        engines = [Engine(b, cfg["vocab"], cfg["heads"], cfg["kv_heads"], cfg["positions"],
                          cfg["block"], 2) for b in (gpu_backend(ctx), cpu_backend(cpu))]
        rng = np.random.default_rng(7 + form)
        p0 = [int(t) for t in rng.integers(0, cfg["vocab"], 2)]
        p1 = [int(t) for t in rng.integers(0, cfg["vocab"], 1)]
        for e in engines:
            e.admit(0, p0, 4)
            e.admit(1, p1, 4)
        outs = [e.step([(0, p0), (1, p1)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1], "prefill")
        t0, t1 = argmax_first(outs[1][0]), argmax_first(outs[1][1])
        outs = [e.step([(0, [t0]), (1, [t1])]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1], "decode")
    finally:
        ctx.close()
        cpu.close()


@pytest.mark.parametrize("hidden", [8192, 16384, 20480])
def test_wide_hidden_norms(torch_gpu, hidden):
    """Residual widths past the 8B and 32B shapes (two q heads, so the projections stay
    small): RMSNorm keeps a thread's 2 (8192) or 4 (16384) float4s of the row in
    registers between its two passes, and at 20480 (5 per thread) reloads the row; the
    layer norms and the head's gathered norm, both precisions, against the CPU path."""
    cfg = dict(layers=1, hidden=hidden, heads=2, kv_heads=1, head_dim=128, ffn=64, vocab=64,
               eps=1e-6, theta=1e6, block=16, positions=64)
    for precision in (0, 1):
        ctx, cpu = make_pair(torch_gpu, cfg, 3, 91 + precision, precision)
        try:
            engines = [Engine(b, cfg["vocab"], cfg["heads"], cfg["kv_heads"], cfg["positions"],
                              cfg["block"], 2) for b in (gpu_backend(ctx), cpu_backend(cpu))]
            rng = np.random.default_rng(hidden + precision)
            p0 = [int(t) for t in rng.integers(0, cfg["vocab"], 3)]
            p1 = [int(t) for t in rng.integers(0, cfg["vocab"], 1)]
            for e in engines:
                e.admit(0, p0, 4)
                e.admit(1, p1, 4)
            outs = [e.step([(0, p0), (1, p1)]) for e in engines]
            check_logits(outs[0], outs[1], [0, 1], "prefill %d" % hidden)
            t0, t1 = argmax_first(outs[1][0]), argmax_first(outs[1][1])
            outs = [e.step([(0, [t0]), (1, [t1])]) for e in engines]
            check_logits(outs[0], outs[1], [0, 1], "decode %d" % hidden)
        finally:
            ctx.close()
            cpu.close()


@pytest.mark.parametrize("form", [0, 1, 2, 3])
def test_wide_chunk_step_with_two_k_groups(torch_gpu, form):
    """Qwen3-8B-wide projections at 100 rows (a 96-token chunk beside four decodes): the
    SwiGLU gate/up (N = 24576) runs 64-row tiles with two k groups per workgroup (its 192
    tiles leave at most one workgroup per CU), QKV, O and down split-K; every form,
    against the CPU path."""
    cfg = dict(WIDE, positions=1024)
    ctx, cpu = make_pair(torch_gpu, cfg, form, 61 + form, 0)
    try:
        engines = [Engine(b, cfg["vocab"], cfg["heads"], cfg["kv_heads"], cfg["positions"],
                          cfg["block"], 5) for b in (gpu_backend(ctx), cpu_backend(cpu))]
        rng = np.random.default_rng(70 + form)
        prompts = [[int(t) for t in rng.integers(0, cfg["vocab"], n)] for n in (5, 9, 3, 7)]
        for e in engines:
            for i, p in enumerate(prompts):
                e.admit(i, p, 4)
        outs = [e.step([(i, p) for i, p in enumerate(prompts)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1, 2, 3], "prefill")
        chunk = [int(t) for t in rng.integers(0, cfg["vocab"], 96)]
        for e in engines:
            e.admit(4, chunk, 4)
        nxt = [argmax_first(outs[1][i]) for i in range(4)]
        outs = [e.step([(i, [nxt[i]]) for i in range(4)] + [(4, chunk)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1, 2, 3, 4], "decodes + chunk of 96")
    finally:
        ctx.close()
        cpu.close()


@pytest.mark.parametrize("form", [3, 0])
def test_long_chunk_step_matches_the_cpu_path(torch_gpu, form):
    """A 150-token chunk beside two decodes: the projections run at M >= 96 (the
    large-M GEMM path for f16 activations, with its f32, residual and SwiGLU
    epilogues) and the chunk's attention at 64-row items."""
    cfg = SMALL
    ctx, cpu = make_pair(torch_gpu, cfg, form, 23, 0)
    try:
        engines = [Engine(b, cfg["vocab"], cfg["heads"], cfg["kv_heads"], cfg["positions"],
                          cfg["block"], 3) for b in (gpu_backend(ctx), cpu_backend(cpu))]
        rng = np.random.default_rng(40 + form)
        p0 = [int(t) for t in rng.integers(0, cfg["vocab"], 9)]
        p1 = [int(t) for t in rng.integers(0, cfg["vocab"], 4)]
        for e in engines:
            e.admit(0, p0, 4)
            e.admit(1, p1, 4)
        outs = [e.step([(0, p0), (1, p1)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1], "prefill")
        p2 = [int(t) for t in rng.integers(0, cfg["vocab"], 150)]
        for e in engines:
            e.admit(2, p2, 4)
        t0, t1 = argmax_first(outs[1][0]), argmax_first(outs[1][1])
        outs = [e.step([(0, [t0]), (1, [t1]), (2, p2)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1, 2], "chunk of 150")
    finally:
        ctx.close()
        cpu.close()


def test_batched_step_equals_the_steps_apart(torch_gpu):
    """batch_test.go:72-200: 1e-5 relative and the same argmax, per sequence."""
    cfg = SMALL
    import tgo_amd
    ctx, cpu = make_pair(torch_gpu, cfg, 3, 5, 1)
    try:
        rng = np.random.default_rng(1)
        prompts = [list(rng.integers(0, cfg["vocab"], n)) for n in (6, 9)]
        e = Engine(gpu_backend(ctx), cfg["vocab"], cfg["heads"], cfg["kv_heads"],
                   cfg["positions"], cfg["block"], 2)
        for i, p in enumerate(prompts):
            e.admit(i, p, 4)
        together = e.step([(0, prompts[0]), (1, prompts[1])])
        # the same two prefills apart (the cache is rewritten identically)
        e2 = Engine(gpu_backend(ctx), cfg["vocab"], cfg["heads"], cfg["kv_heads"],
                    cfg["positions"], cfg["block"], 2)
        for i, p in enumerate(prompts):
            e2.admit(i, p, 4)
        a0 = e2.step([(0, prompts[0])])
        a1 = e2.step([(1, prompts[1])])
        for s, apart in ((0, a0), (1, a1)):
            rel = np.abs(together[s] - apart[s]).max() / np.abs(apart[s]).max()
            assert rel <= 1e-5, (s, rel)
            assert argmax_first(together[s]) == argmax_first(apart[s])
    finally:
        ctx.close()
        cpu.close()


def test_kv_rows_are_the_cast_projections(torch_gpu):
    """nn/attention.go:225-232: K (normed, rotated) and V rows land at slots[t] as f16,
    pad rows (slot = capacity) write nothing."""
    cfg = SMALL
    ctx, cpu = make_pair(torch_gpu, cfg, 0, 3, 1)
    try:
        rng = np.random.default_rng(4)
        e_g = Engine(gpu_backend(ctx), cfg["vocab"], cfg["heads"], cfg["kv_heads"],
                     cfg["positions"], cfg["block"], 2)
        e_c = Engine(cpu_backend(cpu), cfg["vocab"], cfg["heads"], cfg["kv_heads"],
                     cfg["positions"], cfg["block"], 2)
        p = [int(t) for t in rng.integers(0, cfg["vocab"], 10)]
        for e in (e_g, e_c):
            e.admit(0, p, 2)
            e.step([(0, p)])
        torch = torch_gpu
        kp, vp, npos = ctx.kv_pointers()
        n = cfg["layers"] * npos * cfg["kv_heads"] * 128
        dk = torch.empty(n, dtype=torch.int16, device="cuda")
        dv = torch.empty(n, dtype=torch.int16, device="cuda")
        import ctypes
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        torch.cuda.synchronize()
        assert hip.hipMemcpy(ctypes.c_void_p(dk.data_ptr()), ctypes.c_void_p(kp), n * 2, 3) == 0
        assert hip.hipMemcpy(ctypes.c_void_p(dv.data_ptr()), ctypes.c_void_p(vp), n * 2, 3) == 0
        gk = dk.cpu().numpy().view(np.uint16).astype(np.uint16)
        gv = dv.cpu().numpy().view(np.uint16).astype(np.uint16)
        ck, cv = cpu.kv()
        gkf = gk.view(np.float16).astype(np.float32)
        ckf = ck.view(np.float16).astype(np.float32)
        gvf = gv.view(np.float16).astype(np.float32)
        cvf = cv.view(np.float16).astype(np.float32)
        # rows not written are still zero on both sides
        assert np.array_equal(gk == 0, ck == 0) or np.abs(gkf - ckf).max() < 1e-2
        assert np.abs(gkf - ckf).max() <= 2e-3 * np.abs(ckf).max() + 2.0 ** -10
        assert np.abs(gvf - cvf).max() <= 2e-3 * np.abs(cvf).max() + 2.0 ** -10
        assert np.abs(ckf).max() > 0
    finally:
        ctx.close()
        cpu.close()


C1 = dict(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, ffn=3072, vocab=151936,
          eps=1e-6, theta=1e6, block=16, positions=4096)


@pytest.mark.parametrize("gains", ["unit", "seeded"])
@pytest.mark.parametrize("precision", [1, 0])
def test_c1_step_and_64_greedy_steps(torch_gpu, precision, gains):
    """Qwen3-0.6B-shaped, f16 weights N(0,0.02) from a seed; 3 decode
    sequences with contexts {37,300,511} plus a 64-token chunk on a fresh sequence, page 16;
    then 64 greedy steps. Logits within 2e-3 of the CPU path; the device argmax's greedy ids
    identical to the CPU path's. The config states unit gains, and with them every id must
    match. The seeded-gain run binds a distinct non-unit plane to every norm; there an id
    may differ only on a near tie -- the CPU path's top-two margin within twice the row's
    logit error, the reference's reading of a divergence (measure.go:56-66) -- at most
    once, and both sides then take the CPU path's token."""
    cfg = C1
    ctx, cpu = make_pair(torch_gpu, cfg, 0, 2026, precision)
    try:
        if gains == "unit":
            unit_gains(ctx, cpu, cfg)
        V = cfg["vocab"]
        rng = np.random.default_rng(7)
        prompts = [list(rng.integers(0, V, n)) for n in (37, 300, 511)]
        fresh = [int(t) for t in rng.integers(0, V, 64)]
        dev_ids = []
        engines = [Engine(b, V, cfg["heads"], cfg["kv_heads"], cfg["positions"], cfg["block"], 4)
                   for b in (gpu_backend(ctx, dev_ids), cpu_backend(cpu))]
        for e in engines:
            for i, p in enumerate(prompts):
                e.admit(i, p, 80)
        outs = [e.step([(i, p) for i, p in enumerate(prompts)]) for e in engines]
        check_logits(outs[0], outs[1], [0, 1, 2], "contexts")
        toks = [int(t) for t in dev_ids[-1][:3]]
        assert toks == [go_argmax(outs[1][i]) for i in range(3)]
        for e in engines:
            e.admit(3, fresh, 80)
        margins, near = [], []
        work = [(i, [toks[i]]) for i in range(3)] + [(3, fresh)]
        for step in range(65):
            outs = [e.step(work) for e in engines]
            check_logits(outs[0], outs[1], range(4), "step %d" % step)
            g = [int(t) for t in dev_ids[-1]]
            c = [go_argmax(outs[1][i]) for i in range(4)]
            margins.append(min(go_margin(outs[1][i]) for i in range(4)))
            for i in range(4):
                if g[i] == c[i]:
                    continue
                err = float(np.abs(outs[0][i] - outs[1][i]).max())
                assert gains == "seeded" and go_margin(outs[1][i]) <= 2 * err, \
                    ("greedy diverged", step, i, g, c, go_margin(outs[1][i]), err)
                near.append((step, i, go_margin(outs[1][i]), err))
            work = [(i, [c[i]]) for i in range(4)]
        assert len(near) <= 1, near
        print("C1 precision %d, %s gains: min top-2 margin over 65 steps %.3g; near ties %s" %
              (precision, gains, min(margins), near))
    finally:
        ctx.close()
        cpu.close()


@pytest.mark.parametrize("missing", ["wq", "wk", "wv", "wgate", "wup"])
def test_a_step_refuses_a_fused_projection_missing_a_part(torch_gpu, missing):
    """QKV and gate/up are fused device buffers allocated by whichever part is uploaded
    first; a step refuses until every part was uploaded, naming the port, rather than
    running on columns nobody wrote."""
    import tgo_amd
    cfg = SMALL
    ctx = tgo_amd.Context(0)
    try:
        ctx.config(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["kv_heads"],
                   cfg["head_dim"], cfg["ffn"], cfg["vocab"], cfg["eps"], cfg["theta"],
                   cfg["block"])
        ctx.kv_alloc(cfg["positions"])
        d, f, dh = cfg["hidden"], cfg["ffn"], 128
        qw, kw = cfg["heads"] * dh, cfg["kv_heads"] * dh
        rng = np.random.default_rng(3)
        plane = lambda K, N: oracle.f16_bits(rng.standard_normal((K, N)).astype(np.float32) * .02)
        ctx.weight("embed", 0, cfg["vocab"], d, plane(cfg["vocab"], d))
        ctx.weight("lm_head", 0, d, cfg["vocab"], plane(d, cfg["vocab"]))
        ctx.gain("final_norm", np.ones(d, np.float32))
        shapes = dict(wq=(d, qw), wk=(d, kw), wv=(d, kw), wo=(qw, d), wgate=(d, f), wup=(d, f),
                      wdown=(f, d))
        for l in range(cfg["layers"]):
            for name, (K, N) in shapes.items():
                if not (l == 1 and name == missing):
                    ctx.weight("%d.%s" % (l, name), 0, K, N, plane(K, N))
            for gname, w in (("attn_norm", d), ("ffn_norm", d), ("qnorm", dh), ("knorm", dh)):
                ctx.gain("%d.%s" % (l, gname), np.ones(w, np.float32))
        members = [host.Member([1, 2], 0, [0]), host.Member([], 0, [])]
        st = host.new_batch_step(cfg["vocab"], cfg["heads"], cfg["kv_heads"], 2, members,
                                 cfg["block"], cfg["positions"])
        with pytest.raises(tgo_amd.TgoError, match=r"layer 1 has an unbound port \(1\.%s\)"
                           % missing):
            ctx.step(st, host.page_table([[0], []], 1), 1)
        K, N = shapes[missing]
        ctx.weight("1.%s" % missing, 0, K, N, plane(K, N))
        logits, ids, _ = ctx.step(st, host.page_table([[0], []], 1), 1)
        assert np.isfinite(logits).all() and ids[0] >= 0
    finally:
        ctx.close()
