"""TEST INFRASTRUCTURE, NOT PRODUCT.

Pure-Python restatement of tgo's host-side integer logic on the batched path:
batch packing, step assembly, scheduling policy and the prefix block pool.
Small cases only. Each function cites the Go it restates. Only tests/ and
bench.py's cpu_baseline leg may import this.

Parity status: every function here is pinned by the known answers of the
reference's own tests (model/batch_test.go, schedule_test.go,
internal/prefix/prefix_test.go) which tests/golden/ carries as fixtures.
"""
from __future__ import annotations

import hashlib
import math
import struct
from dataclasses import dataclass, field


class Refused(ValueError):
    """A refusal, carrying the field the reference's message names."""


# ---------------------------------------------------------------------------
# model/batch.go:11-159 -- NewBatchStep
# ---------------------------------------------------------------------------

@dataclass
class Member:
    tokens: list
    first: int
    pages: list


def new_batch_step(vocab, heads, kv_heads, rows, members, block, capacity):
    """model.NewBatchStep (model/batch.go:66-152)."""
    if len(members) < 2:
        raise Refused("a batch is two or more sequences")
    if block <= 0:
        raise Refused("addressed through a page table")
    total = sum(len(m.tokens) for m in members)
    if total == 0:
        raise Refused("a step with no rows computes nothing")
    if total > rows:
        raise Refused("member tokens do not fit")
    ids = [0] * rows
    posq = [0] * (rows * heads)
    posk = [0] * (rows * kv_heads)
    slots = [0] * rows
    lengths = [0] * len(members)
    extents = [0] * len(members)
    last = [0] * len(members)
    at, pad = 0, -1
    for i, m in enumerate(members):
        lengths[i] = m.first + len(m.tokens)
        extents[i] = len(m.tokens)
        if m.first < 0:
            raise Refused("a position is not negative")
        if m.tokens:
            pad = i
            last[i] = at + len(m.tokens) - 1
        for j, tok in enumerate(m.tokens):
            if tok < 0 or tok >= vocab:
                raise Refused("outside the model's vocabulary")
            p = m.first + j
            if p // block + 1 > len(m.pages):
                raise Refused("page table entries")
            ids[at] = tok
            slots[at] = m.pages[p // block] * block + p % block
            for h in range(heads):
                posq[at * heads + h] = p
            for h in range(kv_heads):
                posk[at * kv_heads + h] = p
            at += 1
    if at < rows and pad >= 0:
        m = members[pad]
        lastp = m.first + len(m.tokens) - 1
        while at < rows:
            ids[at] = m.tokens[-1]
            slots[at] = capacity
            for h in range(heads):
                posq[at * heads + h] = lastp
            for h in range(kv_heads):
                posk[at * kv_heads + h] = lastp
            at += 1
    return dict(ids=ids, posq=posq, posk=posk, slots=slots, lengths=lengths,
                extents=extents, last=last)


def page_table(pages_per_slot, max_pages):
    """batch.go:397-402: row i is the slot's pages, zero-filled past the lease."""
    table = [0] * (len(pages_per_slot) * max_pages)
    for i, pages in enumerate(pages_per_slot):
        for j, pg in enumerate(pages):
            table[i * max_pages + j] = pg
    return table


def cache_row(pages, block, pos):
    """Physical row of a logical position (model/batch.go:127; plan.go:144-177)."""
    return pages[pos // block] * block + pos % block


# ---------------------------------------------------------------------------
# schedule.go:80-150 -- nextStep, victim
# ---------------------------------------------------------------------------

@dataclass
class SchedState:
    live: bool = False
    prompt: list = field(default_factory=list)
    prefilled: int = 0
    feed: int = 0
    arrived: int = 0


def next_step(slots, chunk, rows):
    """nextStep (schedule.go:80-118). Returns (work [(slot, tokens)], prefill, decode)."""
    if chunk <= 0:
        raise Refused("a chunk is at least one token")
    if rows <= 0:
        raise Refused("carries nothing")
    work, prefill, decode, left = [], 0, 0, rows
    for i, s in enumerate(slots):
        if not s.live or s.prefilled >= len(s.prompt):
            continue
        n = min(chunk, len(s.prompt) - s.prefilled, left)
        if n <= 0:
            continue
        work.append((i, s.prompt[s.prefilled:s.prefilled + n]))
        prefill += n
        left -= n
    for i, s in enumerate(slots):
        if not s.live or s.prefilled < len(s.prompt) or left <= 0:
            continue
        work.append((i, [s.feed]))
        decode += 1
        left -= 1
    work.sort(key=lambda w: w[0])
    return work, prefill, decode


def victim(slots):
    """victim (schedule.go:132-150): last arrived; mid-prefill preferred."""
    best, best_key = -1, 0
    for i, s in enumerate(slots):
        if not s.live:
            continue
        key = s.arrived
        if s.prefilled < len(s.prompt):
            key |= 1 << 63
        if best < 0 or key > best_key:
            best, best_key = i, key
    return best


# ---------------------------------------------------------------------------
# internal/prefix -- hash chain, Pool, Lease
# ---------------------------------------------------------------------------

SCOPE_PROCESS, SCOPE_SESSION, SCOPE_OFF = 0, 1, 2


def chain_seed(scope, domain, salt):
    """seed (internal/prefix/hash.go:28-42)."""
    h = hashlib.sha256()
    h.update(b"tgo/prefix/v1")
    h.update(struct.pack("<Q", scope & 0xFFFFFFFFFFFFFFFF))
    for f in (domain, salt):
        b = f.encode()
        h.update(struct.pack("<Q", len(b)))
        h.update(b)
    return h.digest()


def chain(prev, ids):
    """chain (internal/prefix/hash.go:54-65)."""
    h = hashlib.sha256()
    h.update(prev)
    for i in ids:
        h.update(struct.pack("<Q", int(i) & 0xFFFFFFFFFFFFFFFF))
    return h.digest()


def chain_all(seed, ids, block):
    """chainAll (internal/prefix/hash.go:70-82)."""
    out, prev = [], seed
    for i in range(len(ids) // block):
        prev = chain(prev, ids[i * block:(i + 1) * block])
        out.append(prev)
    return out


class Exhausted(Exception):
    """prefix.ErrExhausted (internal/prefix/prefix.go:54)."""


class Released(Exception):
    """prefix.ErrReleased (internal/prefix/lease.go): the lease was released."""


class Pool:
    """prefix.Pool (internal/prefix/prefix.go:180-461)."""

    def __init__(self, block, blocks, scope=SCOPE_PROCESS):
        if block <= 0 or blocks <= 0:
            raise Refused("block")
        self.block, self.blocks, self.scope = block, blocks, scope
        self.hash = [None] * blocks
        self.published = [False] * blocks
        self.refs = [0] * blocks
        self.entry = {}
        self.free = [blocks - 1 - i for i in range(blocks)]
        self.lru = []  # least recently used first
        self.stats = dict(acquires=0, hits=0, reused=0, prompt=0, evictions=0,
                          publishes=0, adoptions=0)

    def acquire(self, ids, session="", salt="", reserve=0):
        if not ids:
            raise Refused("the prompt is empty")
        if self.scope == SCOPE_SESSION and not session:
            raise Refused("names no session")
        if reserve < 0:
            raise Refused("the reserve is")
        n = len(ids)
        need = (n + reserve + self.block - 1) // self.block
        if need > self.blocks:
            raise Exhausted()
        lease = Lease(self, list(ids))
        domain = session if self.scope == SCOPE_SESSION else ""
        lease.seed = chain_seed(self.scope, domain, salt)
        if self.scope != SCOPE_OFF:
            lease.hashes = chain_all(lease.seed, lease.ids, self.block)
        matched = 0
        limit = (n - 1) // self.block
        while matched < limit and matched < len(lease.hashes):
            bid = self.entry.get(lease.hashes[matched])
            if bid is None:
                break
            self._hold(bid)
            lease.blocks.append(bid)
            matched += 1
        try:
            fresh = self._alloc(need - matched)
        except Exhausted:
            for b in lease.blocks:
                self._drop(b)
            raise
        lease.blocks += fresh
        lease.matched, lease.reused, lease.published = matched, matched * self.block, matched
        self.stats["acquires"] += 1
        self.stats["prompt"] += n
        self.stats["reused"] += lease.reused
        if matched:
            self.stats["hits"] += 1
        return lease

    def _alloc(self, n):
        out = []
        while len(out) < n:
            bid = self._take()
            if bid is None:
                for b in out:
                    self.refs[b] = 0
                    self.free.append(b)
                raise Exhausted()
            out.append(bid)
        return out

    def _take(self):
        if self.free:
            bid = self.free.pop()
            self.refs[bid] = 1
            return bid
        if not self.lru:
            return None
        bid = self.lru.pop(0)
        del self.entry[self.hash[bid]]
        self.hash[bid], self.published[bid] = None, False
        self.stats["evictions"] += 1
        self.refs[bid] = 1
        return bid

    def _hold(self, bid):
        self.refs[bid] += 1
        if self.refs[bid] == 1:
            self.lru.remove(bid)

    def _drop(self, bid):
        self.refs[bid] -= 1
        if self.refs[bid] > 0:
            return
        if self.published[bid]:
            self.lru.append(bid)
            return
        self.free.append(bid)

    def counts(self):
        in_use = sum(1 for r in self.refs if r > 0)
        return dict(in_use=in_use, cached=len(self.lru), free=len(self.free))


class Lease:
    """prefix.Lease (internal/prefix/lease.go:14-222)."""

    def __init__(self, pool, ids):
        self.pool, self.ids = pool, ids
        self.blocks, self.hashes = [], []
        self.seed = b""
        self.matched = self.reused = self.published = 0
        self.released = False

    def row(self, t):
        return self.blocks[t // self.pool.block] * self.pool.block + t % self.pool.block

    def grow(self, n):
        p = self.pool
        if self.released:
            raise Released()
        if n == 0:
            return
        want = (len(self.ids) + n + p.block - 1) // p.block
        if want > p.blocks:
            raise Exhausted()
        k = want - len(self.blocks)
        if k > 0:
            self.blocks += p._alloc(k)

    def commit(self, ids):
        p = self.pool
        if self.released:
            raise Released()
        if not ids:
            return
        want = (len(self.ids) + len(ids) + p.block - 1) // p.block
        if want > len(self.blocks):
            raise Refused("grow it before the step")
        self.ids += list(ids)
        if p.scope != SCOPE_OFF:
            prev = self.hashes[-1] if self.hashes else self.seed
            for i in range(len(self.hashes), len(self.ids) // p.block):
                prev = chain(prev, self.ids[i * p.block:(i + 1) * p.block])
                self.hashes.append(prev)

    def publish(self, written):
        p = self.pool
        if self.released or p.scope == SCOPE_OFF:
            return list(self.blocks)
        complete = written // p.block
        i = self.published
        while i < len(self.hashes) and i < complete:
            h, mine = self.hashes[i], self.blocks[i]
            theirs = p.entry.get(h)
            if theirs is not None:
                if theirs != mine:
                    p._hold(theirs)
                    p._drop(mine)
                    self.blocks[i] = theirs
                    p.stats["adoptions"] += 1
                self.published = i + 1
                i += 1
                continue
            p.entry[h] = mine
            p.hash[mine], p.published[mine] = h, True
            p.stats["publishes"] += 1
            self.published = i + 1
            i += 1
        return list(self.blocks)

    def release(self):
        if self.released:
            return
        self.released = True
        for b in self.blocks:
            self.pool._drop(b)


# ---------------------------------------------------------------------------
# scheduler.go:34-397 + batch.go:235-458 -- Scheduler over a Batch
# ---------------------------------------------------------------------------

class Scheduler:
    """tgo.Scheduler (scheduler.go) over a Batch (batch.go) and a prefix Pool, with the
    forward pass left to `backend(ports, table, max_pages) -> logits [B, V]` (the CPU
    restatement in the tests). Admit takes the first free slot and leases the prompt plus
    its reserve (batch.go:235-262, scheduler.go:184-222); step asks nextStep for the
    work, grows each worker's lease (batchSlot.reserve, batch.go:555-575), packs every
    slot as a member (batch.go:349-360) with NewBatchStep at exactly the rows the work
    holds (tgo rounds rows up to a bucket, plan.go:66-77; the padding rows are inert),
    runs the step, then commits and publishes each worker's blocks (batchSlot.commit,
    batch.go:577-589) and advances the books (scheduler.go:343-357). The page table is
    the pool-wide one (batch.go:397-402): pool blocks wide, zero past each lease."""

    def __init__(self, n, chunk, reserve, rows, block, blocks, vocab, heads, kv_heads,
                 backend):
        if reserve <= 0:
            raise Refused("the scheduler's reserve")
        if n < 2:
            raise Refused("a batch is two or more")
        self.chunk = chunk or 512  # DefaultChunk (schedule.go:21)
        self.reserve, self.rows, self.block = reserve, rows, block
        self.V, self.H, self.Hkv = vocab, heads, kv_heads
        self.capacity = blocks * block
        self.max_pages = blocks
        self.pool = Pool(block, blocks)
        self.state = [SchedState() for _ in range(n)]
        self.lease = [None] * n
        self.length = [0] * n
        self.next = 0
        self.backend = backend
        self.last = None  # (ports, table) of the last step

    def admit(self, prompt, reserve=0):
        reserve = reserve or self.reserve
        free = next((i for i, s in enumerate(self.state) if not s.live), -1)
        if free < 0:
            raise Exhausted()
        self._release(free)
        lease = self.pool.acquire(list(prompt), reserve=reserve)
        self.lease[free], self.length[free] = lease, lease.reused
        self.next += 1
        self.state[free] = SchedState(True, list(prompt), lease.reused, 0, self.next)
        return free

    def _release(self, slot):
        if self.lease[slot] is not None:
            self.lease[slot].release()
        self.lease[slot], self.length[slot] = None, 0

    def finish(self, slot):
        self._release(slot)
        self.state[slot] = SchedState()

    def evict(self):
        v = victim(self.state)
        if v >= 0:
            self.finish(v)
        return v

    def feed(self, slot, token):
        s = self.state[slot]
        if not s.live or s.prefilled < len(s.prompt):
            raise Refused("a token fed before the prompt is scored")
        s.feed = token
        s.prompt.append(token)
        s.prefilled += 1

    def step(self):
        """-> ([(slot, logits row, done)], prefill tokens, decodes)."""
        work, prefill, decode = next_step(self.state, self.chunk, self.rows)
        if not work:
            return [], prefill, decode
        members = [Member([], self.length[i], list(l.blocks) if l else [])
                   for i, l in enumerate(self.lease)]
        for slot, toks in work:
            lease = self.lease[slot]
            need = self.length[slot] + len(toks)
            if need > len(lease.ids):
                lease.grow(need - len(lease.ids))
            members[slot] = Member(list(toks), self.length[slot], list(lease.blocks))
        total = sum(len(t) for _, t in work)
        ports = new_batch_step(self.V, self.H, self.Hkv, total, members, self.block,
                               self.capacity)
        table = page_table([m.pages for m in members], self.max_pages)
        self.last = (ports, table)
        logits = self.backend(ports, table, self.max_pages)
        out = []
        for slot, toks in work:
            lease = self.lease[slot]
            need = self.length[slot] + len(toks)
            if need > len(lease.ids):
                lease.commit(list(toks[len(toks) - (need - len(lease.ids)):]))
            lease.publish(self.length[slot] + len(toks))
            self.length[slot] += len(toks)
            st = self.state[slot]
            if st.prefilled < len(st.prompt):
                st.prefilled += len(toks)
            out.append((slot, logits[slot], st.prefilled >= len(st.prompt)))
        return out, prefill, decode


# ---------------------------------------------------------------------------
# reference test fixtures
# ---------------------------------------------------------------------------

def spread(n, seed):
    """spread (internal/conformance/ragged_test.go:121-128), as float32."""
    import numpy as np
    out = np.empty(n, dtype=np.float32)
    for i in range(n):
        x = float((i * seed) % 97) / 97.0
        out[i] = np.float32(math.sin(6.0 * x) * (0.5 + x))
    return out


def f16exact(seed):
    """f16exact (model/graph_rig_test.go:42-55): a multiple of 1/8 in [-2,2)."""
    seed &= 0xFFFFFFFF
    seed ^= (seed << 13) & 0xFFFFFFFF
    seed ^= seed >> 17
    seed ^= (seed << 5) & 0xFFFFFFFF
    return float(int(seed % 32) - 16) / 8.0


def rsqrt_f32(dh):
    """session.go:821-823: 1/sqrt(d_h) rounded once from float64 to float32."""
    import numpy as np
    return float(np.float32(1.0 / math.sqrt(dh)))


def argmax_first(row):
    """sample/stages.go:196-206: index of the first strict maximum."""
    best, bi = None, -1
    for i, v in enumerate(row):
        if best is None or v > best:
            best, bi = v, i
    return bi


def top_two_margin(row):
    """TopTwoMargin (internal/conformance/measure.go:91-110): the largest logit minus
    the second largest, in float64, seeded with row[0], row[1] and folded with strict
    comparisons. Fewer than two logits is a binding mistake and refused."""
    if len(row) < 2:
        raise Refused("TopTwoMargin over fewer than two logits")
    first, second = float(row[0]), float(row[1])
    if second > first:
        first, second = second, first
    for x in row[2:]:
        v = float(x)
        if v > first:
            first, second = v, first
        elif v > second:
            second = v
    return first - second
