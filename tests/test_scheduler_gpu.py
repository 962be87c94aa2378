"""The library's Scheduler on the GPU: steps with posq/posk/slots derived on
the device, and overlap mode (submit / collect) against the synchronous step.

* A step whose posq, posk and slots are left to the device gives the same
  logits, to the bit, as the same step with NewBatchStep's packed ports
  (model.NewBatchStep, batch.go:310-340, restated in oracle/host.py), padding
  rows included. The derived rows also take their rotary cos and sin from the
  table computed once per step, the packed ports from the angles computed in
  the q/k-norm + RoPE kernel: the two agree to the bit.
* Overlap mode runs the steps the synchronous scheduler runs when the caller
  admits and retires the same sequences before each submit as before each
  step. Each sequence's greedy tokens are then identical: a row's result does
  not depend on the rows beside it at a given step size, and the attention of
  a sequence is the same mixed or apart (ragged_test.go:295).
"""
import numpy as np
import pytest

import tgo_amd
from oracle import host

pytestmark = pytest.mark.gpu

CFG = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1024,
           eps=1e-6, theta=1e6, block=4, positions=1024)


def new_ctx(torch, form=3, seed=21):
    c = CFG
    ctx = tgo_amd.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    ctx.config(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"],
               c["vocab"], c["eps"], c["theta"], c["block"])
    ctx.synth_weights(seed, form, 0.02)
    ctx.kv_alloc(c["positions"])
    return ctx


def packed_step(rng, rows_pad, shape=((13, 13), (0, 0), (9, 1))):
    """Members (by default a prefill chunk, an idle one and a decode; (prompt, new) tokens
    each) packed by NewBatchStep, plus rows_pad padding rows."""
    c = CFG
    pool = host.Pool(c["block"], c["positions"] // c["block"])
    members = []
    for n_prompt, n_new in shape:
        if n_prompt == 0:
            members.append(host.Member([], 0, []))
            continue
        toks = [int(t) for t in rng.integers(0, c["vocab"], n_prompt)]
        lease = pool.acquire(toks, reserve=4)  # blocks for the prompt and 4 more
        first = n_prompt - n_new
        members.append(host.Member(toks[first:], first, list(lease.blocks)))
    rows = sum(len(m.tokens) for m in members) + rows_pad
    st = host.new_batch_step(c["vocab"], c["heads"], c["kv_heads"], rows, members, c["block"],
                             c["positions"])
    max_pages = c["positions"] // c["block"]
    table = host.page_table([m.pages for m in members], max_pages)
    return st, table, max_pages


@pytest.mark.parametrize("rows_pad", [0, 3])
def test_derived_ports_equal_the_packed_ports(torch_gpu, rows_pad):
    torch = torch_gpu
    st, table, max_pages = packed_step(np.random.default_rng(5), rows_pad)
    a, b = new_ctx(torch), new_ctx(torch)
    la, aa, _ = a.step(st, table, max_pages)
    derived = dict(st, posq=None, posk=None, slots=None)
    lb, ab, _ = b.step(derived, table, max_pages)
    assert np.isfinite(la).all()
    assert np.array_equal(la, lb)
    assert np.array_equal(aa, ab)
    # the idle member (extent 0): zero logits and no token
    assert not la[1].any() and aa[1] == -1
    assert la[0].any() and la[2].any() and aa[0] >= 0 and aa[2] >= 0
    # the KV pools the two steps wrote, every layer (padding rows write nothing)
    torch.cuda.synchronize()
    pools = [pool_copy(x) for x in (a, b)]
    assert np.array_equal(pools[0], pools[1])
    assert np.count_nonzero(pools[0]) > 0
    a.close()
    b.close()


def test_fused_qkv_epilogue_equals_the_separate_kernel(torch_gpu):
    """69 rows (a 48-token chunk, an idle member, a decode, a 20-token chunk after 10 cached
    positions): the QKV projection runs on the pipelined exact kernel, unsplit with one k
    group (K = 256), so with derived rows it does q/k-norm, RoPE and the K/V write in its
    epilogue, while packed ports take the separate qk_rope_kv_kernel. Both compute every
    value the same way: logits, tokens and both KV pools equal to the bit."""
    torch = torch_gpu
    st, table, max_pages = packed_step(np.random.default_rng(9), 0,
                                       ((48, 48), (0, 0), (9, 1), (30, 20)))
    assert len(st["ids"]) == 69
    a, b = new_ctx(torch), new_ctx(torch)
    la, aa, _ = a.step(st, table, max_pages)
    lb, ab, _ = b.step(dict(st, posq=None, posk=None, slots=None), table, max_pages)
    assert np.isfinite(la).all() and la[0].any() and la[3].any()
    assert np.array_equal(la, lb)
    assert np.array_equal(aa, ab)
    torch.cuda.synchronize()
    pools = [pool_copy(x) for x in (a, b)]
    assert np.array_equal(pools[0], pools[1])
    assert np.count_nonzero(pools[0]) > 0
    a.close()
    b.close()


def pool_copy(ctx):
    """Both KV pools of every layer, copied to the host as f16 bits."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    k, v, positions = ctx.kv_pointers()
    n = CFG["layers"] * positions * CFG["kv_heads"] * CFG["head_dim"]
    out = np.empty((2, n), np.uint16)
    for i, src in enumerate((k, v)):
        assert hip.hipMemcpy(out[i].ctypes.data, src, n * 2, 2) == 0  # device to host
    return out


class Driver:
    """Arrivals and retirements around a scheduler: at most `target` live sequences, each
    retired after `budget` generated tokens. The decisions after a step depend only on
    which slots produced a token, so they can be taken before the step is read back."""

    def __init__(self, sched, seed, target, count):
        rng = np.random.default_rng(seed)
        V = CFG["vocab"]
        self.queue = [([int(t) for t in rng.integers(0, V, int(rng.integers(3, 21)))],
                       int(rng.integers(2, 9))) for _ in range(count)]
        self.sched, self.target = sched, target
        self.seq_of, self.made, self.budget = {}, {}, {}
        self.next_seq = 0
        self.admit()

    def admit(self):
        while self.sched.live() < self.target and self.queue:
            prompt, budget = self.queue.pop(0)
            slot = self.sched.admit(prompt, reserve=budget + 1)
            self.seq_of[slot] = self.next_seq
            self.made[slot], self.budget[slot] = 0, budget
            self.next_seq += 1

    def decide(self, produced, tokens=None):
        """produced: [(slot, done)]; tokens (sync mode): {slot: token} to feed."""
        for slot, done in produced:
            if not done:
                continue
            self.made[slot] += 1
            if self.made[slot] >= self.budget[slot]:
                self.sched.finish(slot)
                del self.seq_of[slot]
            elif tokens is not None:
                self.sched.feed(slot, tokens[slot])
        self.admit()


def run_sync(sched, steps):
    d = Driver(sched, 3, 5, 30)
    streams, sizes = {}, []
    for _ in range(steps):
        produced, pf, dc, _ = sched.step()
        sizes.append((pf, dc))
        toks = {}
        for slot, tok, done in produced:
            if done:
                streams.setdefault(d.seq_of[slot], []).append(tok)
                toks[slot] = tok
        d.decide([(s, dn) for s, _, dn in produced], toks)
    return streams, sizes


def run_overlap(sched, steps):
    sched.set_overlap(True)
    d = Driver(sched, 3, 5, 30)
    streams, sizes = {}, []
    labels = []  # per step in flight: {slot: sequence} when it was submitted
    info, pf, dc = sched.submit()
    sizes.append((pf, dc))
    labels.append(dict(d.seq_of))
    d.decide(info)
    for k in range(steps):
        if k + 1 < steps:
            nxt, pf, dc = sched.submit()
            sizes.append((pf, dc))
            labels.append(dict(d.seq_of))
        produced, _ = sched.collect()
        seqs = labels.pop(0)
        for slot, tok, done in produced:
            if done:
                streams.setdefault(seqs[slot], []).append(tok)
        if k + 1 < steps:
            d.decide(nxt)
    assert sched.collect()[0] == []  # nothing left in flight
    return streams, sizes


def test_overlap_mode_runs_the_synchronous_steps(torch_gpu):
    """Also twice over, each in a context of its own opened after the last one closed:
    the second run starts on memory the first released and must not see its state."""
    torch = torch_gpu
    steps = 40
    a, b = new_ctx(torch), new_ctx(torch)
    sa = tgo_amd.Scheduler(a, 8, chunk=8, reserve=4, max_rows=64)
    sb = tgo_amd.Scheduler(b, 8, chunk=8, reserve=4, max_rows=64)
    sync_streams, sync_sizes = run_sync(sa, steps)
    ov_streams, ov_sizes = run_overlap(sb, steps)
    assert sync_sizes == ov_sizes
    assert len(sync_streams) >= 10
    assert sync_streams == ov_streams
    sa.close()
    sb.close()
    a.close()
    b.close()
    for _ in range(2):
        c = new_ctx(torch)
        sc = tgo_amd.Scheduler(c, 8, chunk=8, reserve=4, max_rows=64)
        again, again_sizes = run_overlap(sc, steps)
        sc.close()
        c.close()
        assert again_sizes == sync_sizes
        assert again == sync_streams


def test_overlap_refusals(torch_gpu):
    torch = torch_gpu
    ctx = new_ctx(torch)
    s = tgo_amd.Scheduler(ctx, 4, chunk=8, reserve=4, max_rows=64)
    with pytest.raises(tgo_amd.TgoError, match="overlap mode"):
        s.submit()
    slot = s.admit([1, 2, 3], reserve=8)
    s.set_overlap(True)
    with pytest.raises(tgo_amd.TgoError, match="tgohip_sched_submit"):
        s.step()
    info, _, _ = s.submit()
    assert info == [(slot, True)]
    with pytest.raises(tgo_amd.TgoError, match="feeds each generated token itself"):
        s.feed(slot, 7)
    with pytest.raises(tgo_amd.TgoError, match="in flight"):
        s.set_overlap(False)
    s.submit()
    with pytest.raises(tgo_amd.TgoError, match="two steps are in flight"):
        s.submit()
    with pytest.raises(tgo_amd.TgoError, match="a step is in flight"):
        s.last_step()
    # a slot finished with rows in flight is not reused until they land
    s.finish(slot)
    with pytest.raises(tgo_amd.TgoError):
        for _ in range(4):
            s.admit([5, 6], reserve=2)
    out1, _ = s.collect()
    out2, _ = s.collect()
    assert [o[0] for o in out1] == [slot] and [o[0] for o in out2] == [slot]
    assert out2[0][1] >= 0
    s.set_overlap(False)
    s.close()
    ctx.close()


def test_profile_times_every_kth_layer(torch_gpu):
    """tgohip_set_profile(ctx, k) brackets the attention launch of every k-th layer: the
    launch count and the algorithmic bytes follow k, and a negative k is refused."""
    torch = torch_gpu
    st, table, max_pages = packed_step(np.random.default_rng(9), 0)
    ctx = new_ctx(torch)
    counts = {}
    for k in (1, 2):
        ctx.set_profile(True, k)
        for _ in range(3):
            ctx.step(st, table, max_pages)
        ms, nbytes, launches = ctx.profile_read()
        counts[k] = (launches, nbytes)
        assert ms > 0
    ctx.set_profile(False)
    assert counts[1][0] == 3 * CFG["layers"]
    assert counts[2][0] == 3 * ((CFG["layers"] + 1) // 2)
    assert counts[1][1] / counts[1][0] == counts[2][1] / counts[2][0]
    with pytest.raises(tgo_amd.TgoError, match="layer stride"):
        ctx.set_profile(True, -1)
    ctx.close()


# ---- the library Scheduler against the reference's, restated ------------------------
#
# oracle/host.py's Scheduler restates scheduler.go over Batch.step (batch.go:314-458) and a
# prefix Pool, with the forward pass on the CPU restatement. The library's Scheduler
# (tgohip_sched_*, the driver of bench.py) and it are given the same admissions, feeds,
# finishes and evictions; every step's ports must be equal to the bit (the page table row
# by row: the library's stride is the step's longest lease, the reference's the pool's) and
# the greedy tokens equal.

def prompt_ids(seed, n, vocab):
    """promptIDs (prefixcache_test.go:33-43): a 32-bit xorshift stream over [1, vocab)."""
    out, x = [], (seed * 2654435761 + 1) & 0xFFFFFFFF
    for _ in range(n):
        x ^= (x << 13) & 0xFFFFFFFF
        x ^= x >> 17
        x ^= (x << 5) & 0xFFFFFFFF
        out.append(1 + x % (vocab - 1))
    return out


class Pair:
    """The library Scheduler on the GPU and the oracle Scheduler on the CPU path."""

    def __init__(self, torch, n, chunk, reserve, max_rows, form=3, seed=21):
        import oracle
        c = CFG
        self.ctx = new_ctx(torch, form, seed)
        self.lib = tgo_amd.Scheduler(self.ctx, n, chunk=chunk, reserve=reserve,
                                     max_rows=max_rows)
        self.cpu = oracle.CPUModel(c["layers"], c["hidden"], c["heads"], c["kv_heads"],
                                   c["head_dim"], c["ffn"], c["vocab"], c["eps"], c["theta"],
                                   c["block"], c["positions"])
        self.cpu.synth(seed, form, 0.02)
        self.orc = host.Scheduler(n, chunk, reserve, max_rows, c["block"],
                                  c["positions"] // c["block"], c["vocab"], c["heads"],
                                  c["kv_heads"], lambda st, tb, mp: self.cpu.step(st, tb, mp))
        self.near = 0

    def close(self):
        self.lib.close()
        self.ctx.close()
        self.cpu.close()

    def admit(self, prompt, reserve=0):
        a = self.lib.admit(prompt, reserve)
        b = self.orc.admit(prompt, reserve)
        assert a == b, ("admit took different slots", a, b)
        assert self.lib.length(a) == self.orc.length[a]  # the prefix pool's reuse
        return a

    def finish(self, slot):
        self.lib.finish(slot)
        self.orc.finish(slot)

    def evict(self):
        a, b = self.lib.evict(), self.orc.evict()
        assert a == b
        return a

    def step(self):
        """One step on both; checks the ports, the books and the tokens and feeds the
        tokens. -> ([(slot, token, done)], prefill, decodes)."""
        got, pf, dc, _ = self.lib.step()
        want, pf2, dc2 = self.orc.step()
        assert (pf, dc) == (pf2, dc2)
        assert [(s, d) for s, _, d in got] == [(s, d) for s, _, d in want]
        if not got:
            return [], pf, dc
        st, pages, maxp = self.lib.last_step()
        ost, otable = self.orc.last
        for k in ("ids", "posq", "posk", "slots", "lengths", "extents", "last"):
            assert np.array_equal(np.asarray(st[k], np.uint32), np.asarray(ost[k], np.uint32)), k
        B, omax = len(ost["lengths"]), self.orc.max_pages
        lt = np.asarray(pages, np.uint32).reshape(B, maxp)
        ot = np.asarray(otable, np.uint32).reshape(B, omax)
        assert np.array_equal(lt, ot[:, :maxp]) and not ot[:, maxp:].any()
        out = []
        for (slot, tok, done), (_, logits, _) in zip(got, want):
            if done:
                cpu_tok = int(np.argmax(logits))
                if tok != cpu_tok:  # only a near tie may flip
                    top = np.sort(logits.astype(np.float64))[-2:]
                    assert top[1] - top[0] <= 1e-3 * np.abs(logits).max(), (slot, tok, cpu_tok)
                    self.near += 1
                self.lib.feed(slot, cpu_tok)
                self.orc.feed(slot, cpu_tok)
                tok = cpu_tok
            out.append((slot, tok, done))
        return out, pf, dc


def test_a_chunk_and_the_decodes_run_in_one_dispatch(torch_gpu):
    """scheduler_test.go:41-113 on the library Scheduler, checked step by step against the
    reference's Scheduler restated: prompts of 6 and 5 are one step of 11 prefill tokens
    (the chunk of 8 is per sequence); a 20-token prompt admitted beside the two decoders is
    chunked in the same dispatch (8 prefill tokens + 2 decodes) and is not sampleable."""
    V = CFG["vocab"]
    p = Pair(torch_gpu, 3, 8, 32, 64)
    try:
        for i, prompt in enumerate((prompt_ids(2, 6, V), prompt_ids(3, 5, V))):
            assert p.admit(prompt) == i
        out, pf, dc = p.step()
        assert (pf, dc) == (11, 0) and all(d for _, _, d in out)
        slot = p.admit(prompt_ids(1, 20, V))
        out, pf, dc = p.step()
        assert (pf, dc) == (8, 2) and len(out) == 3
        assert [d for s, _, d in out if s == slot] == [False]
        for _ in range(3):  # the long prompt finishes: 8 + 4, then decodes
            out, pf, dc = p.step()
        assert (pf, dc) == (0, 3)
    finally:
        p.close()


def test_a_schedulers_decodes_match_the_sessions_they_batch(torch_gpu):
    """scheduler_test.go:115-190: two prompts (6 and 10 tokens, chunk 8) stepped together
    for six steps, feeding greedy tokens, generate what each generates alone."""
    V = CFG["vocab"]
    prompts = [prompt_ids(4, 6, V), prompt_ids(5, 10, V)]

    def run(which):
        p = Pair(torch_gpu, 2, 8, 32, 64)
        try:
            for i in which:
                p.admit(prompts[i])
            made = {i: [] for i in which}
            slot_of = {s: i for s, i in enumerate(which)}
            for _ in range(6):
                out, _, _ = p.step()
                for s, tok, done in out:
                    if done:
                        made[slot_of[s]].append(tok)
            return made
        finally:
            p.close()

    together = run([0, 1])
    for i in (0, 1):
        alone = run([i])[i]
        assert together[i] and together[i][:len(alone)] == alone[:len(together[i])], i


def test_the_library_scheduler_runs_the_reference_schedulers_steps(torch_gpu):
    """A seeded walk of 60 steps: admissions (prompts that share an 8-token prefix, so the
    pool reuses published blocks), feeds, finishes and evictions, the same on both sides;
    every step's ports bit-exact and every greedy token equal."""
    V = CFG["vocab"]
    rng = np.random.default_rng(17)
    p = Pair(torch_gpu, 6, 8, 4, 40)
    common = prompt_ids(9, 8, V)
    made = {}
    try:
        steps = 0
        for it in range(60):
            live = [s for s in range(6) if p.orc.state[s].live]
            if len(live) < 6 and rng.random() < 0.5:
                n = int(rng.integers(3, 24))
                prompt = (common if rng.random() < 0.5 else []) + \
                    [int(t) for t in rng.integers(0, V, n)]
                s = p.admit(prompt, reserve=int(rng.integers(4, 16)))
                made[s] = 0
            decoding = [s for s in live if p.orc.state[s].prefilled >= len(p.orc.state[s].prompt)]
            if decoding and rng.random() < 0.2:
                s = int(rng.choice(decoding))
                p.finish(s)
            if live and rng.random() < 0.05:
                p.evict()
            out, _, _ = p.step()
            steps += bool(out)
            for s, _, done in out:
                if done:
                    made[s] = made.get(s, 0) + 1
                    if made[s] >= 12:  # the reserve is spent: retire it
                        p.finish(s)
        assert steps >= 40 and p.near <= 1
        assert p.orc.pool.stats["hits"] > 0 and p.orc.pool.stats["reused"] > 0
    finally:
        p.close()
