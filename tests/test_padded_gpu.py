"""tgo's bucket-padded step on the GPU against tgo's CPU path restated (orc_model_step).

Batch.step rounds a step's rows up to a bucket (batch.go:362-366, plan.go:66-77) and
model.NewBatchStep fills the rows past the members' with the last member's last token at
its last position and slot = capacity (model/batch.go:140-150). Those rows must not write
K/V (plan.go:180-192: a slot at or past capacity is a dropped write), attention leaves
them inert, and nobody reads their logits. Checked here:

* logits of every member that worked within 2e-3 of the CPU row's largest |logit|, and
  greedy ids identical (outside near ties at the C4 width, as in test_config_gpu);
* every pool row that no member's slot names is exactly what it was before the step, on
  the GPU and on the CPU path, in every layer (the small model starts from a zeroed pool,
  so those rows are zero); the rows the members name match the CPU path's;
* the padded step equals the same step packed without padding, to the bit: the library
  computes only the members' rows when the padding cannot change anything;
* a padding row whose slot lies in the pool (ports not packed by NewBatchStep) does write
  its K/V, as the reference's ScatterRows would, and the step still matches the CPU path.
"""
import numpy as np
import pytest

import bench
import oracle
import tgo_amd
from oracle import host

pytestmark = pytest.mark.gpu

CFG = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1024,
           eps=1e-6, theta=1e6, block=4, positions=1024)


def small_ctx(torch, seed):
    c = CFG
    ctx = tgo_amd.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    ctx.config(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"],
               c["vocab"], c["eps"], c["theta"], c["block"])
    ctx.synth_weights(seed, tgo_amd.FORM_I4_SYM, 0.02)
    ctx.kv_alloc(c["positions"])
    return ctx


def small_cpu(seed):
    c = CFG
    cpu = oracle.CPUModel(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"],
                          c["ffn"], c["vocab"], c["eps"], c["theta"], c["block"], c["positions"])
    cpu.synth(seed, tgo_amd.FORM_I4_SYM, 0.02)
    return cpu


def gpu_pool(ctx, layers, kv_heads):
    """[2 (K, V), layers, positions, kv_heads * 128] f16 bits of the device pools."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    k, v, positions = ctx.kv_pointers()
    out = np.empty((2, layers, positions, kv_heads * 128), np.uint16)
    for i, src in enumerate((k, v)):
        assert hip.hipMemcpy(out[i].ctypes.data, src, out[i].nbytes, 2) == 0  # device to host
    return out


def cpu_pool(cpu, layers, kv_heads, positions):
    k, v = cpu.kv()
    return np.stack([np.asarray(k).reshape(layers, positions, kv_heads * 128),
                     np.asarray(v).reshape(layers, positions, kv_heads * 128)])


def f16(bits):
    return bits.view(np.float16).astype(np.float32)


def check_pools(gpu_after, cpu_after, before, named, what):
    """Rows no slot names: unchanged on both sides, to the bit. Named rows: the CPU
    path's f16 K/V within 2e-3 of the row's largest magnitude plus 2^-10."""
    other = np.ones(gpu_after.shape[2], bool)
    other[list(named)] = False
    for side, pool in (("gpu", gpu_after), ("cpu", cpu_after)):
        assert np.array_equal(pool[:, :, other], before[:, :, other]), (what, side, "untouched rows")
    idx = sorted(named)
    g, c = f16(gpu_after[:, :, idx]), f16(cpu_after[:, :, idx])
    bound = 2e-3 * np.abs(c).max(axis=-1, keepdims=True) + 2.0 ** -10
    assert (np.abs(g - c) <= bound).all(), (what, "named rows", float(np.abs(g - c).max()))


def pad_ports(st, rows, capacity):
    """NewBatchStep's padding of an unpadded step out to `rows` (model/batch.go:140-150):
    the last member that worked repeats its last token at its last position, slot =
    capacity. An unpadded step's last claimed row is that member's last row."""
    n = len(st["ids"])
    H = len(st["posq"]) // n
    Hkv = len(st["posk"]) // n
    last = n - 1
    out = {k: list(v) for k, v in st.items()}
    out["ids"] += [st["ids"][last]] * (rows - n)
    out["posq"] += [st["posq"][last * H]] * ((rows - n) * H)
    out["posk"] += [st["posk"][last * Hkv]] * ((rows - n) * Hkv)
    out["slots"] += [capacity] * (rows - n)
    return out


def small_members(rng):
    """A 13-token prefill chunk, an idle member and a one-token decode at position 8."""
    c = CFG
    pool = host.Pool(c["block"], c["positions"] // c["block"])
    members = []
    for n_prompt, n_new in ((13, 13), (0, 0), (9, 1)):
        if n_prompt == 0:
            members.append(host.Member([], 0, []))
            continue
        toks = [int(t) for t in rng.integers(0, c["vocab"], n_prompt)]
        lease = pool.acquire(toks, reserve=4)
        first = n_prompt - n_new
        members.append(host.Member(toks[first:], first, list(lease.blocks)))
    return members


def compare_logits(got, ids, want, extents, what, allow_near=False):
    for b, n in enumerate(extents):
        if n == 0:
            assert ids[b] == -1 and not got[b].any(), (what, b)
            continue
        rowmax = float(np.abs(want[b]).max())
        err = float(np.abs(got[b] - want[b]).max())
        assert err <= 2e-3 * rowmax, (what, b, err, rowmax)
        w = int(np.argmax(want[b]))
        if int(ids[b]) != w:
            top = np.sort(want[b].astype(np.float64))[-2:]
            assert allow_near and top[1] - top[0] <= 2 * err, (what, "greedy differs", b)


def test_bucket_padded_step_matches_the_cpu_path(torch_gpu):
    """14 rows of work in a 32-row bucket (batch.go:362-366; plan.go:31's first rung)."""
    torch = torch_gpu
    c, seed = CFG, 31
    members = small_members(np.random.default_rng(7))
    claimed = sum(len(m.tokens) for m in members)
    assert claimed == 14
    mk = lambda rows: host.new_batch_step(c["vocab"], c["heads"], c["kv_heads"], rows, members,
                                          c["block"], c["positions"])
    padded, exact = mk(32), mk(claimed)
    assert padded["slots"][claimed:] == [c["positions"]] * (32 - claimed)
    max_pages = c["positions"] // c["block"]
    table = host.page_table([m.pages for m in members], max_pages)
    named = {s for s in padded["slots"][:claimed]}

    a, b, d = small_ctx(torch, seed), small_ctx(torch, seed), small_ctx(torch, seed)
    cpu = small_cpu(seed)
    try:
        la, ia, _ = a.step(padded, table, max_pages)
        lb, ib, _ = b.step(exact, table, max_pages)
        ld, idd, _ = d.step(dict(padded, posq=None, posk=None, slots=None), table, max_pages)
        torch.cuda.synchronize()
        assert np.array_equal(la, lb) and np.array_equal(ia, ib), "padded != unpadded"
        assert np.array_equal(la, ld) and np.array_equal(ia, idd), "derived != packed"
        want = cpu.step(padded, table, max_pages)
        compare_logits(la, ia, want, padded["extents"], "padded 14 -> 32")
        zero = np.zeros((2, c["layers"], c["positions"], c["kv_heads"] * 128), np.uint16)
        pa = gpu_pool(a, c["layers"], c["kv_heads"])
        pc = cpu_pool(cpu, c["layers"], c["kv_heads"], c["positions"])
        check_pools(pa, pc, zero, named, "padded 14 -> 32")
        assert np.array_equal(pa, gpu_pool(b, c["layers"], c["kv_heads"]))
        assert np.array_equal(pa, gpu_pool(d, c["layers"], c["kv_heads"]))
    finally:
        cpu.close()
        for x in (a, b, d):
            x.close()


def test_padding_row_inside_the_pool_writes_its_kv(torch_gpu):
    """Ports not packed by NewBatchStep: padding row 20 names a free pool row. The
    reference's ScatterRows writes it (only slots at or past capacity are dropped), so
    every row runs and that row holds the padding row's K/V, as on the CPU path."""
    torch = torch_gpu
    c, seed = CFG, 32
    members = small_members(np.random.default_rng(8))
    st = host.new_batch_step(c["vocab"], c["heads"], c["kv_heads"], 32, members, c["block"],
                             c["positions"])
    max_pages = c["positions"] // c["block"]
    table = host.page_table([m.pages for m in members], max_pages)
    named = {s for s in st["slots"][:14]}
    free = max(named) + 37
    assert free < c["positions"] and free not in named
    st["slots"][20] = free
    named.add(free)
    a, cpu = small_ctx(torch, seed), small_cpu(seed)
    try:
        la, ia, _ = a.step(st, table, max_pages)
        torch.cuda.synchronize()
        want = cpu.step(st, table, max_pages)
        compare_logits(la, ia, want, st["extents"], "pad row in the pool")
        zero = np.zeros((2, c["layers"], c["positions"], c["kv_heads"] * 128), np.uint16)
        pa = gpu_pool(a, c["layers"], c["kv_heads"])
        check_pools(pa, cpu_pool(cpu, c["layers"], c["kv_heads"], c["positions"]), zero, named,
                    "pad row in the pool")
        assert pa[:, :, free].any(), "the padding row's K/V was not written"
    finally:
        cpu.close()
        a.close()


@pytest.mark.timeout(900)
def test_c4_step_bucketed_to_2048_rows_matches_the_cpu_path(torch_gpu):
    """bench.py's C4 step (130 members, 1152 rows, 8B widths, int4, two layers deep, tgo's
    f32 arithmetic: precision mode 1) padded to the 2048-row rung of tgo's bucket ladder."""
    from test_config_gpu import copy_pool, cpu_model, open_ctx
    torch = torch_gpu
    cfg, form, pool = bench.C4, tgo_amd.FORM_I4_SYM, bench.POOL
    layers = 2
    ctx = open_ctx(cfg, form, pool, bench.SEED)
    ctx.set_precision(1)
    cpu = None
    try:
        wl = bench.Workload(tgo_amd, ctx, bench.SEED)
        ctx.kv_synth(bench.SEED, 1.0, min(pool, wl.used_positions + 64 * bench.CHUNK))
        wl.sched.step()  # writes this step's K/V: replaying it below rewrites the same values
        st, pages, maxp = wl.sched.last_step()
        assert len(st["ids"]) == 1152
        padded = pad_ports(st, 2048, pool)
        named = {s for s in st["slots"]}
        before = gpu_pool(ctx, layers, cfg["kv_heads"])
        cpu = cpu_model(cfg, form, pool, bench.SEED)
        copy_pool(ctx, cpu, layers, cfg["kv_heads"], pool)
        lp, ip, _ = ctx.step(padded, pages, maxp)
        after = gpu_pool(ctx, layers, cfg["kv_heads"])
        assert np.array_equal(after, before), "the replayed padded step changed the pool"
        lu, iu, _ = ctx.step(st, pages, maxp)
        assert np.array_equal(lp, lu) and np.array_equal(ip, iu), "padded != unpadded"
        want = cpu.step(padded, pages, maxp, layers=layers)
        compare_logits(lp, ip, want, st["extents"], "C4 bucketed to 2048", allow_near=True)
        check_pools(after, cpu_pool(cpu, layers, cfg["kv_heads"], pool), before, named,
                    "C4 bucketed to 2048")
    finally:
        if cpu:
            cpu.close()
        ctx.close()


def test_step_margins_cover_the_last_step_only(torch_gpu):
    """tgohip_step_margins returns the last step's members: after a 3-member step, a
    2-member step leaves 2 margins to read, and asking for 3 is refused instead of
    returning the earlier step's third."""
    torch = torch_gpu
    c = CFG
    members = small_members(np.random.default_rng(9))
    max_pages = c["positions"] // c["block"]
    ctx = small_ctx(torch, 33)
    try:
        st3 = host.new_batch_step(c["vocab"], c["heads"], c["kv_heads"], 14, members, c["block"],
                                  c["positions"])
        ctx.step(st3, host.page_table([m.pages for m in members], max_pages), max_pages)
        assert len(ctx.step_margins(3)) == 3
        two = [members[0], members[2]]
        st2 = host.new_batch_step(c["vocab"], c["heads"], c["kv_heads"], 14, two, c["block"],
                                  c["positions"])
        logits, _, _ = ctx.step(st2, host.page_table([m.pages for m in two], max_pages), max_pages)
        mg = ctx.step_margins(2)
        for b in range(2):
            top = np.sort(logits[b].astype(np.float64))[-2:]
            assert mg[b] == top[1] - top[0]
        with pytest.raises(tgo_amd.TgoError, match="last step held 2"):
            ctx.step_margins(3)
    finally:
        ctx.close()
