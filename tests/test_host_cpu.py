"""The product's host logic (libtgohip.so through its C ABI) against the reference's
own known answers and against the oracle's host restatement: batch packing
(model/batch_test.go), the scheduler's policy (schedule_test.go), the prefix block
pool (internal/prefix/*_test.go), SHA-256, and the load-time conversions. Also that
the library loads and exports every symbol the header declares. CPU only: no call
here touches a GPU."""
import hashlib
import json
import os
import re

import numpy as np
import pytest

import oracle
from oracle import host
import tgo_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_known_answers.json")))
V_SYNTH = 112  # the synthetic config's vocabulary (model/graph_rig_test.go:21-24)


def test_library_exports_every_declared_symbol():
    text = open(os.path.join(ROOT, "include", "tgohip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = sorted(set(re.findall(r"\b(tgohip_[a-z0-9_]+)\s*\(", text)))
    assert len(names) > 40
    lib = tgo_amd.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert tgo_amd.lib().tgohip_version()


# ---- model.NewBatchStep ---------------------------------------------------------

def both_new_batch_step(vocab, heads, kv_heads, rows, members, block, capacity):
    """Run the product and the oracle; each returns dict or the refusal message."""
    out = []
    try:
        out.append(tgo_amd.new_batch_step(vocab, heads, kv_heads, rows,
                                          [(m["tokens"], m["first"], m["pages"]) for m in members],
                                          block, capacity))
    except tgo_amd.TgoError as e:
        out.append(str(e))
    try:
        out.append(host.new_batch_step(vocab, heads, kv_heads, rows,
                                       [host.Member(m["tokens"], m["first"], m["pages"])
                                        for m in members], block, capacity))
    except host.Refused as e:
        out.append(str(e))
    return out


def test_batch_step_pads_and_addresses_known_answer():
    g = GOLD["batch_pads"]
    prod, orc = both_new_batch_step(V_SYNTH, 2, 1, g["rows"], g["members"], g["block"],
                                    g["capacity"])
    for st in (prod, orc):
        assert list(st["extents"]) == g["want_extents"]
        assert list(st["lengths"]) == g["want_lengths"]
        assert list(st["last"]) == g["want_last"]
        assert list(st["slots"][:3]) == g["want_slots_prefix"]
        assert all(s == g["want_pad_slot"] for s in st["slots"][3:])
    for k in orc:
        assert list(prod[k]) == list(orc[k]), k


@pytest.mark.parametrize("case", GOLD["batch_refusals"]["cases"], ids=lambda c: c["name"])
def test_batch_step_refusals_name_the_field(case):
    members = GOLD["batch_refusals"]["sound"] if case["members"] == "sound" else case["members"]
    if case["name"] == "one member":
        members = members[:1]
    members = [dict(m, tokens=[V_SYNTH if t == "V" else t for t in m["tokens"]]) for m in members]
    prod, orc = both_new_batch_step(V_SYNTH, 2, 1, case["rows"], members, case["block"], 64)
    assert isinstance(prod, str) and case["want"] in prod, prod
    assert isinstance(orc, str)


def test_batch_step_random_members_agree_with_the_oracle():
    rng = np.random.default_rng(11)
    for trial in range(200):
        B = int(rng.integers(2, 6))
        block = int(rng.choice([1, 2, 4, 16]))
        members = []
        for i in range(B):
            n = int(rng.integers(0, 6))
            first = int(rng.integers(0, 40))
            npg = (first + n + block - 1) // block
            if rng.random() < 0.05:
                npg = max(npg - 1, 0)  # a table that does not reach
            members.append(dict(tokens=[int(t) for t in rng.integers(0, V_SYNTH + 1 * (rng.random() < 0.03), n)],
                                first=first, pages=[int(p) for p in rng.permutation(64)[:npg]]))
        total = sum(len(m["tokens"]) for m in members)
        rows = total + int(rng.integers(-1, 5))
        prod, orc = both_new_batch_step(V_SYNTH, 4, 2, rows, members, block, 64 * block)
        assert isinstance(prod, str) == isinstance(orc, str), (trial, prod, orc)
        if not isinstance(prod, str):
            for k in orc:
                assert list(prod[k]) == list(orc[k]), (trial, k)


# ---- schedule.go: nextStep, victim ------------------------------------------------

def states(rows):
    """[prompt_len, prefilled, feed, arrived] rows -> oracle slot states."""
    return [host.SchedState(live=True, prompt=list(range(p)), prefilled=f, feed=fd, arrived=a)
            for p, f, fd, a in rows]


def product_next(sl, chunk, rows):
    return tgo_amd.next_step([1 if s.live else 0 for s in sl], [len(s.prompt) for s in sl],
                             [s.prefilled for s in sl], chunk, rows)


def test_schedule_known_answers():
    g = GOLD["schedule"]
    c = g["chunk_rides"]
    sl = states(c["slots"])
    work, pf, dc = product_next(sl, c["chunk"], c["rows"])
    assert (pf, dc, len(work), sum(w[2] for w in work)) == \
        (c["want_prefill"], c["want_decode"], c["want_work"], c["want_tokens"])
    owork, opf, odc = host.next_step(sl, c["chunk"], c["rows"])
    assert (opf, odc, len(owork)) == (pf, dc, len(work))
    for plen, chunk, rows, want in g["chunk_caps"]:
        sl = states([[plen, 0, 0, 1]])
        work, pf, dc = product_next(sl, chunk, rows)
        assert pf == want and work == [(0, 0, want)]
        assert host.next_step(sl, chunk, rows)[1] == want
    pfirst = g["prefill_first"]
    for rows, want_pf, want_dc in pfirst["cases"]:
        sl = states(pfirst["slots"])
        _, pf, dc = product_next(sl, pfirst["chunk"], rows)
        assert (pf, dc) == (want_pf, want_dc)
        assert host.next_step(sl, pfirst["chunk"], rows)[1:] == (want_pf, want_dc)
    lo = g["left_out"]
    _, pf, dc = product_next(states(lo["slots"]), lo["chunk"], lo["rows"])
    assert dc == lo["want_decode"] and pf == 0
    for v in g["victims"]:
        sl = states(v["slots"])
        assert host.victim(sl) == v["want"]
        assert tgo_amd.victim([1] * len(sl), [len(s.prompt) for s in sl],
                              [s.prefilled for s in sl], [s.arrived for s in sl]) == v["want"]


def test_schedule_refusals():
    for chunk, rows in ((0, 4), (4, 0)):
        with pytest.raises(tgo_amd.TgoError):
            tgo_amd.next_step([1], [3], [0], chunk, rows)
        with pytest.raises(host.Refused):
            host.next_step(states([[3, 0, 0, 1]]), chunk, rows)


def test_schedule_random_states_agree_with_the_oracle():
    rng = np.random.default_rng(12)
    for trial in range(500):
        n = int(rng.integers(0, 9))
        sl = []
        for i in range(n):
            p = int(rng.integers(1, 3000))
            f = p if rng.random() < 0.6 else int(rng.integers(0, p + 1))
            sl.append(host.SchedState(live=bool(rng.random() < 0.8), prompt=list(range(p)),
                                      prefilled=f, feed=int(rng.integers(0, 100)),
                                      arrived=int(rng.integers(0, 1 << 40))))
        chunk = int(rng.choice([1, 7, 512]))
        rows = int(rng.integers(1, 1200))
        work, pf, dc = product_next(sl, chunk, rows)
        owork, opf, odc = host.next_step(sl, chunk, rows)
        assert (pf, dc) == (opf, odc), trial
        want = [(i, sl[i].prefilled if sl[i].prefilled < len(sl[i].prompt) else -1,
                 len(toks)) for i, toks in owork]
        assert work == want, trial
        assert tgo_amd.victim([1 if s.live else 0 for s in sl], [len(s.prompt) for s in sl],
                              [s.prefilled for s in sl], [s.arrived for s in sl]) == host.victim(sl)


# ---- internal/prefix: hash chain -------------------------------------------------

def test_sha256_matches_hashlib():
    rng = np.random.default_rng(13)
    for n in [0, 1, 55, 56, 63, 64, 65, 119, 120, 1000, 4096 + 17]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert tgo_amd.sha256(data) == hashlib.sha256(data).digest(), n


def run_ids(start, n):
    return list(range(start, start + n))


def test_hash_chain_known_properties():
    """hash_test.go:8-66 and scope_test.go:116-127 on the oracle's chain."""
    s = host.chain_seed(host.SCOPE_PROCESS, "", "")
    shared = run_ids(9000, 4)
    first = host.chain_all(s, run_ids(100, 4) + shared, 4)
    second = host.chain_all(s, run_ids(500, 4) + shared, 4)
    assert first[0] != second[0] and first[1] != second[1]
    assert host.chain_all(s, run_ids(100, 4) + shared, 4)[1] == first[1]
    assert len(host.chain_all(s, run_ids(100, 3), 4)) == 0
    assert len(host.chain_all(s, run_ids(100, 9), 4)) == 2
    assert host.chain(s, [1, 23]) != host.chain(s, [12, 3])
    assert host.chain(s, [0, 0]) != host.chain(s, [0])
    plain = host.chain_all(s, run_ids(100, 12), 4)
    salted = host.chain_all(host.chain_seed(host.SCOPE_PROCESS, "", "tenant-7"), run_ids(100, 12), 4)
    assert all(a != b for a, b in zip(plain, salted))
    assert host.chain_seed(0, "", "pepper") == host.chain_seed(0, "", "pepper")
    assert host.chain_seed(0, "", "pepper") != host.chain_seed(1, "", "pepper")


# ---- internal/prefix: Pool and Lease, both implementations -----------------------

class ExhaustedE(Exception):
    pass


class RefusedE(Exception):
    pass


class ReleasedE(Exception):
    pass


class OracleImpl:
    name = "oracle"

    def __init__(self, block, blocks, scope=0):
        self.p = host.Pool(block, blocks, scope)

    def acquire(self, ids, session="", salt="", reserve=0):
        try:
            return OracleLease(self.p.acquire(list(ids), session, salt, reserve))
        except host.Exhausted:
            raise ExhaustedE()
        except host.Refused:
            raise RefusedE()

    def stats(self):
        s = dict(self.p.stats)
        s.update(self.p.counts())
        return s

    def close(self):
        pass


class OracleLease:
    def __init__(self, l):
        self.l = l

    def blocks(self):
        return list(self.l.blocks)

    def reused(self):
        return self.l.reused

    def matched(self):
        return self.l.matched

    def len(self):
        return len(self.l.ids)

    def append(self, *ids):
        try:
            self.l.grow(len(ids))
            self.l.commit(list(ids))
        except host.Exhausted:
            raise ExhaustedE()
        except host.Released:
            raise ReleasedE()

    def publish(self, written):
        return self.l.publish(written)

    def row(self, t):
        return self.l.row(t)

    def release(self):
        self.l.release()


class ProductImpl:
    name = "product"

    def __init__(self, block, blocks, scope=0):
        self.p = tgo_amd.Pool(block, blocks, scope)
        self.block = block

    def acquire(self, ids, session="", salt="", reserve=0):
        try:
            return ProductLease(self.p.acquire(list(ids), session, salt, reserve), self.block)
        except tgo_amd.TgoError as e:
            if e.code == tgo_amd.EEXHAUSTED:
                raise ExhaustedE(str(e))
            raise RefusedE(str(e))

    def stats(self):
        return self.p.stats()

    def close(self):
        self.p.close()


class ProductLease:
    def __init__(self, l, block):
        self.l, self.block = l, block

    def blocks(self):
        return self.l.blocks()

    def reused(self):
        return self.l.reused()

    def matched(self):
        return self.l.reused() // self.block

    def len(self):
        return self.l.len()

    def append(self, *ids):
        try:
            self.l.grow(len(ids))
            self.l.commit(list(ids))
        except tgo_amd.TgoError as e:
            if e.code == tgo_amd.EEXHAUSTED:
                raise ExhaustedE(str(e))
            if e.code == tgo_amd.ESTATE:
                raise ReleasedE(str(e))
            raise

    def publish(self, written):
        return self.l.publish(written)

    def row(self, t):
        b = self.blocks()
        return b[t // self.block] * self.block + t % self.block

    def release(self):
        self.l.release()


IMPLS = [OracleImpl, ProductImpl]
TB, TBS = 4, 7  # testBlock, testBlocks (prefix_test.go:15-18)


@pytest.fixture(params=IMPLS, ids=lambda c: c.name)
def mk(request):
    made = []

    def make(block=TB, blocks=TBS, scope=0):
        p = request.param(block, blocks, scope)
        made.append(p)
        return p
    yield make
    for p in made:
        p.close()


def warm(p, ids, **kw):
    l = p.acquire(ids, **kw)
    l.publish(l.len())
    l.release()


def test_warm_prefix_reused_cold_not(mk):
    p = mk()
    prompt = run_ids(100, 9)
    cold = p.acquire(prompt)
    assert cold.reused() == 0
    cold.publish(cold.len())
    cold.release()
    w = p.acquire(prompt)
    assert w.reused() == 8 and w.matched() == 2
    assert w.blocks()[:2] == cold.blocks()[:2]
    w.release()
    warm(p, run_ids(100, 9))
    assert p.acquire(run_ids(500, 9)).reused() == 0


def test_interior_run_is_not_shared(mk):
    p = mk(32, 7)
    shared = run_ids(9000, 32)
    first = run_ids(100, 32) + shared + [700]
    second = run_ids(500, 32) + shared + [700]
    one = p.acquire(first)
    theirs = one.publish(one.len())
    one.release()
    l = p.acquire(second)
    assert l.matched() == 0
    mine = l.blocks()
    page = l.publish(l.len())
    assert p.stats()["adoptions"] == 0
    assert page == mine and theirs[0] not in page and theirs[1] not in page
    assert p.acquire(first).matched() == 2


def test_resubmission_prefills_one_token_and_full_hit_gives_up_a_block(mk):
    p = mk()
    prompt = run_ids(100, 9)
    warm(p, prompt)
    l = p.acquire(prompt)
    assert l.reused() == 8
    l.release()
    p = mk()
    prompt = run_ids(100, 8)
    warm(p, prompt)
    l = p.acquire(prompt)
    assert l.reused() == TB
    before = l.blocks()
    after = l.publish(l.len())
    assert before[1] != after[1]
    assert p.stats()["adoptions"] == 1
    l.release()
    s = p.stats()
    assert s["cached"] == 2 and s["free"] == TBS - 2


def test_hit_is_block_aligned(mk):
    p = mk()
    warm(p, run_ids(100, 7) + run_ids(300, 4))
    l = p.acquire(run_ids(100, 7) + run_ids(800, 4))
    assert l.reused() == TB


def test_evicted_prefix_is_a_miss(mk):
    p = mk(TB, 3)
    victim = run_ids(100, 5)
    warm(p, victim)
    assert p.stats()["cached"] == 1
    pressure = p.acquire(run_ids(500, 3 * TB))
    assert p.stats()["evictions"] > 0
    pressure.publish(pressure.len())
    pressure.release()
    assert p.acquire(victim).matched() == 0


def test_shared_block_survives_and_pressure_is_refused(mk):
    p = mk()
    prompt = run_ids(100, 9)
    a = p.acquire(prompt)
    a.publish(a.len())
    b = p.acquire(prompt)
    assert b.matched() == 2
    a.release()
    with pytest.raises(ExhaustedE):
        p.acquire(run_ids(900, TBS * TB))
    s = p.stats()
    assert s["in_use"] == 3
    b.release()


def test_eviction_never_frees_a_referenced_block(mk):
    p = mk(TB, 3)
    held = p.acquire(run_ids(100, 3 * TB))
    with pytest.raises(ExhaustedE):
        p.acquire(run_ids(500, 1))
    s = p.stats()
    assert (s["in_use"], s["evictions"], s["free"]) == (3, 0, 0)
    held.release()


def test_lru_order(mk):
    p = mk(TB, 3)
    warm(p, run_ids(100, TB))
    warm(p, run_ids(500, TB))
    assert p.stats()["cached"] == 2
    l = p.acquire(run_ids(900, TB + 1))
    l.release()
    assert p.stats()["evictions"] == 1
    k = p.acquire(run_ids(500, TB) + [1])
    assert k.matched() == 1
    k.release()
    assert p.acquire(run_ids(100, TB) + [1]).matched() == 0
    p = mk(TB, 3)
    warm(p, run_ids(100, TB))
    warm(p, run_ids(500, TB))
    warm(p, run_ids(100, TB))
    p.acquire(run_ids(900, TB + 1)).release()
    assert p.acquire(run_ids(100, TB) + [1]).matched() == 1


def test_stats_count_what_the_pool_did(mk):
    p = mk()
    prompt = run_ids(100, 9)
    warm(p, prompt)
    p.acquire(prompt).release()
    s = p.stats()
    assert (s["acquires"], s["hits"], s["prompt"], s["reused"], s["publishes"]) == (2, 1, 18, 8, 2)
    assert (s["in_use"], s["cached"], s["free"]) == (0, 2, TBS - 2)


def test_refusals(mk):
    p = mk()
    with pytest.raises(RefusedE):
        p.acquire([])
    with pytest.raises(RefusedE):
        p.acquire([1], reserve=-1)
    with pytest.raises(RefusedE):
        mk(TB, TBS, 1).acquire(run_ids(100, 5))
    with pytest.raises(ExhaustedE):
        mk(TB, 3).acquire(run_ids(100, 3 * TB + 1))


def test_pool_construction_refusals():
    for block, blocks, scope, want in ((0, 3, 0, "at least one position"),
                                       (-8, 3, 0, "at least one position"),
                                       (4, 0, 0, "at least one"), (4, 3, 9, "is not a scope")):
        with pytest.raises(tgo_amd.TgoError, match=want):
            tgo_amd.Pool(block, blocks, scope)


def test_refused_acquire_gives_back_what_it_matched(mk):
    p = mk(TB, 3)
    prefix = run_ids(100, TB + 1)
    warm(p, prefix)
    hog = p.acquire(run_ids(500, 2 * TB))
    s = p.stats()
    assert (s["free"], s["cached"]) == (0, 1)
    with pytest.raises(ExhaustedE):
        p.acquire(run_ids(100, TB) + run_ids(900, 2 * TB))
    s = p.stats()
    assert (s["cached"], s["in_use"], s["free"]) == (1, 2, 0)
    hog.release()
    assert p.acquire(prefix).matched() == 1


def test_reserve_held_from_admission_and_rounded_once(mk):
    p = mk(4, 4)
    l = p.acquire([1, 2, 3, 4], reserve=8)
    assert len(l.blocks()) == 3 and p.stats()["in_use"] == 3
    l.append(5, 6, 7, 8)
    assert p.stats()["in_use"] == 3
    with pytest.raises(ExhaustedE):
        p.acquire([9, 10], reserve=8)
    l.release()
    p = mk(4, 8)
    l = p.acquire([1, 2], reserve=2)
    assert len(l.blocks()) == 1


def test_lease_rows_and_growth(mk):
    p = mk()
    churn = p.acquire(run_ids(500, 3 * TB))
    pin = p.acquire(run_ids(700, 1))
    churn.release()
    l = p.acquire(run_ids(100, 9))
    b = l.blocks()
    assert b != list(range(len(b))) and l.row(0) != 0
    for pos, want in ((0, b[0] * TB), (3, b[0] * TB + 3), (4, b[1] * TB), (7, b[1] * TB + 3),
                      (8, b[2] * TB)):
        assert l.row(pos) == want
    l.release()
    pin.release()
    p = mk()
    l = p.acquire(run_ids(100, 5))
    assert len(l.blocks()) == 2
    l.append(1, 2, 3)
    assert len(l.blocks()) == 2 and l.len() == 8
    l.append(4)
    assert len(l.blocks()) == 3 and l.row(8) == l.blocks()[2] * TB
    l.append()
    assert l.len() == 9


def test_append_publish_and_reuse_next_turn(mk):
    p = mk()
    l = p.acquire(run_ids(100, 5))
    l.publish(l.len())
    assert p.stats()["publishes"] == 1
    l.append(700, 701, 702)
    assert len(l.blocks()) == 2
    l.publish(l.len())
    assert p.stats()["publishes"] == 2
    l.release()
    p = mk()
    prompt = run_ids(100, 5)
    l = p.acquire(prompt)
    l.publish(l.len())
    l.append(700, 701, 702, 703)
    l.publish(l.len())
    l.release()
    assert p.stats()["publishes"] == 2
    turn = p.acquire(prompt + [700, 701, 702, 703, 900])
    assert (turn.matched(), turn.reused()) == (2, 8)


def test_append_refusals(mk):
    p = mk(TB, 3)
    l = p.acquire(run_ids(100, 2 * TB))
    l.append(1, 2, 3, 4)
    assert len(l.blocks()) == 3 and l.len() == 3 * TB
    l.publish(l.len())
    assert p.stats()["publishes"] == 3
    with pytest.raises(ExhaustedE):
        l.append(5)
    assert l.len() == 3 * TB
    l.release()
    p = mk(TB, 3)
    mine = p.acquire(run_ids(100, TB))
    p.acquire(run_ids(500, 2 * TB))
    with pytest.raises(ExhaustedE):
        mine.append(1)
    assert mine.len() == TB and len(mine.blocks()) == 1
    p = mk()
    l = p.acquire(run_ids(100, 5))
    l.release()
    with pytest.raises(ReleasedE):
        l.append(1)
    assert len(l.publish(l.len())) == 2 and p.stats()["publishes"] == 0


def test_release_idempotent_and_publish_twice(mk):
    p = mk()
    prompt = run_ids(100, 9)
    a = p.acquire(prompt)
    a.publish(a.len())
    b = p.acquire(prompt)
    a.release()
    a.release()
    assert p.stats()["in_use"] == 3
    b.release()
    p = mk()
    l = p.acquire(run_ids(100, 9))
    assert l.publish(l.len()) == l.publish(l.len())
    assert p.stats()["publishes"] == 2
    l.release()
    s = p.stats()
    assert (s["cached"], s["free"]) == (2, TBS - 2)


def test_scopes(mk):
    p = mk(TB, TBS, 1)
    prompt = run_ids(100, 9)
    warm(p, prompt, session="alice")
    assert p.acquire(prompt, session="bob").matched() == 0
    assert p.acquire(prompt, session="alice").matched() == 2
    p = mk(TB, TBS, 1)
    warm(p, prompt, session="a", salt="b")
    assert p.acquire(prompt, session="ab").matched() == 0
    p = mk()
    warm(p, prompt, salt="tenant-7")
    for salt in ("", "tenant-9"):
        l = p.acquire(prompt, salt=salt)
        assert l.matched() == 0
        l.release()
    assert p.acquire(prompt, salt="tenant-7").matched() == 2
    p = mk(TB, TBS, 2)
    warm(p, prompt)
    l = p.acquire(prompt)
    assert (l.matched(), l.reused(), len(l.blocks())) == (0, 0, 3)
    s = p.stats()
    assert (s["publishes"], s["cached"]) == (0, 0)
    l.release()
    assert p.stats()["free"] == TBS
    l = p.acquire(run_ids(100, 5))
    l.append(1, 2, 3, 4)
    assert len(l.blocks()) == 3 and p.stats()["publishes"] == 0


def test_pool_random_operations_agree_with_the_oracle():
    """A seeded random walk of acquire / append / publish / release with shared prefixes,
    sessions and salts: every lease's page table, reuse and every counter agree after
    every operation (the concurrent_test.go accounting invariant included)."""
    for seed in range(20):
        rng = np.random.default_rng(100 + seed)
        block, blocks, scope = int(rng.choice([2, 4, 16])), int(rng.integers(3, 40)), \
            int(rng.choice([0, 0, 1, 2]))
        o, q = OracleImpl(block, blocks, scope), ProductImpl(block, blocks, scope)
        bases = [[int(x) for x in rng.integers(0, 50, 64)] for _ in range(4)]
        live = []
        try:
            for step in range(300):
                op = rng.random()
                if op < 0.4 or not live:
                    base = bases[int(rng.integers(0, 4))]
                    n = int(rng.integers(1, 40))
                    ids = base[:min(n, 64)] + [int(x) for x in rng.integers(0, 50, max(0, n - 64))]
                    if rng.random() < 0.3:
                        ids = ids + [int(rng.integers(0, 50))]
                    kw = dict(session=str(rng.integers(0, 2)) if scope == 1 else "",
                              salt=["", "s"][int(rng.integers(0, 2))],
                              reserve=int(rng.integers(0, 8)))
                    res = []
                    for impl in (o, q):
                        try:
                            res.append(impl.acquire(ids, **kw))
                        except ExhaustedE:
                            res.append("exhausted")
                    assert (res[0] == "exhausted") == (res[1] == "exhausted"), (seed, step)
                    if res[0] != "exhausted":
                        live.append(res)
                elif op < 0.6:
                    lo, lq = live[int(rng.integers(0, len(live)))]
                    add = [int(x) for x in rng.integers(0, 50, int(rng.integers(0, 6)))]
                    r = []
                    for l in (lo, lq):
                        try:
                            l.append(*add)
                            r.append("ok")
                        except (ExhaustedE, ReleasedE) as e:
                            r.append(type(e).__name__)
                    assert r[0] == r[1], (seed, step, r)
                elif op < 0.8:
                    lo, lq = live[int(rng.integers(0, len(live)))]
                    w = int(rng.integers(0, lo.len() + 1))
                    assert lo.publish(w) == lq.publish(w), (seed, step)
                else:
                    i = int(rng.integers(0, len(live)))
                    lo, lq = live.pop(i)
                    lo.release()
                    lq.release()
                so, sq = o.stats(), q.stats()
                assert so == {k: sq[k] for k in so}, (seed, step, so, sq)
                assert so["in_use"] + so["cached"] + so["free"] == blocks
                for lo, lq in live:
                    assert lo.blocks() == lq.blocks() and lo.reused() == lq.reused()
                    assert lo.len() == lq.len()
        finally:
            q.close()


# ---- weights/convert.go at load ----------------------------------------------------

def test_load_conversions_are_bit_exact_with_the_oracle():
    rng = np.random.default_rng(14)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 3,
                        np.asarray([65504, 65505, 1e30, -1e30, np.inf, -np.inf, np.nan, 3e-5,
                                    -3e-5, 6.103515625e-05, 0.0, -0.0], np.float32)])
    got, sat = tgo_amd.to_f16(x)
    want = oracle.f16_bits(x)
    assert np.array_equal(got, want)
    assert sat == int(np.sum((np.abs(x) > 65504) & ~np.isnan(x)))
    w = (rng.standard_normal(32 * 999 + 5) * 0.1).astype(np.float32)
    q, s = tgo_amd.quantize_int8(w)
    oq, os_ = np.empty(w.size, np.int8), np.empty((w.size + 31) // 32, np.uint16)
    oracle.lib.orc_quantize_int8(oracle.ptr(w), w.size, oracle.ptr(oq), oracle.ptr(os_))
    assert np.array_equal(q, oq) and np.array_equal(s, os_)
    c, s, z = tgo_amd.quantize_int4(w)
    oc = np.empty((w.size + 7) // 8, np.uint32)
    osc, oz = np.empty((w.size + 127) // 128, np.uint16), np.empty((w.size + 127) // 128, np.uint16)
    oracle.lib.orc_quantize_int4_tgo(oracle.ptr(w), w.size, oracle.ptr(oc), oracle.ptr(osc),
                                     oracle.ptr(oz))
    assert np.array_equal(c, oc) and np.array_equal(s, osc) and np.array_equal(z, oz)


def test_oracle_scheduler_known_answers():
    """oracle/host.py's Scheduler against scheduler_test.go:41-113's counts (a dummy forward
    pass): 6 + 5 prompts under a chunk of 8 are one step of 11 prefill tokens; a 20-token
    prompt joins two decoders as 8 prefill tokens + 2 decodes and is not sampleable; then
    8 + 2, 4 + 2 and 3 decodes. Admission takes the first free slot; Admit refuses without
    one; victim is the last arrival, mid-prefill first."""
    import numpy as np
    calls = []

    def backend(st, table, max_pages):
        calls.append((len(st["ids"]), len(st["lengths"]), max_pages, len(table)))
        return np.zeros((len(st["lengths"]), 64), np.float32)

    s = host.Scheduler(3, 8, 32, 64, 4, 64, 64, 4, 2, backend)
    assert s.admit(list(range(1, 7))) == 0 and s.admit(list(range(7, 12))) == 1
    out, pf, dc = s.step()
    assert (pf, dc) == (11, 0) and [(o[0], o[2]) for o in out] == [(0, True), (1, True)]
    assert calls[-1] == (11, 3, 64, 3 * 64)
    s.feed(0, 5)
    s.feed(1, 6)
    assert s.admit(list(range(20, 40))) == 2
    seen = []
    for _ in range(4):
        out, pf, dc = s.step()
        seen.append((pf, dc, [(o[0], o[2]) for o in out]))
        for slot, _, done in out:
            if done:
                s.feed(slot, 1)
    assert seen == [(8, 2, [(0, True), (1, True), (2, False)]),
                    (8, 2, [(0, True), (1, True), (2, False)]),
                    (4, 2, [(0, True), (1, True), (2, True)]),
                    (0, 3, [(0, True), (1, True), (2, True)])]
    with pytest.raises(host.Exhausted):
        s.admit([1, 2])
    assert s.evict() == 2  # the last arrival
    s.finish(0)
    assert s.admit([1, 2, 3]) == 0
    assert s.evict() == 0 and s.evict() == 1 and s.evict() == -1
