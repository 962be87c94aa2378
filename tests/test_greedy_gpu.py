"""The device greedy selection (tgohip_greedy: argmax_part_kernel + argmax_final_kernel)
on crafted rows, against the Go loops it restates, run on the host (oracle/host.py):

  * argmax (sample/stages.go:196-206): best = x[0], then i taken only when x[i] > best --
    the first index of the maximum, a NaN never taken after index 0, 0 when x[0] is NaN;
  * TopTwoMargin (internal/conformance/measure.go:91-110): seeded with x[0], x[1], later
    values taken by strict comparison, the difference in float64.

Both bit-exact (ids equal; margins equal as float64, NaN where Go gives NaN). The rows
cover the reference's known answers (tests/golden), ties, NaN at index 0, 1 and later,
+-inf, all-equal rows, V not a multiple of 4, V = 2 and the C4 vocabulary with the
maximum at chunk and stride edges, and batches whose rows split over 1 to 16 workgroups."""
import json
import math
import os

import numpy as np
import pytest

from oracle import host

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_known_answers.json")))
nan, inf = float("nan"), float("inf")


def run(ctx, torch, rows):
    V = len(rows[0])
    x = torch.tensor(np.asarray(rows, np.float32), device="cuda")
    ids = torch.full((len(rows),), -7, dtype=torch.int32, device="cuda")
    mg = torch.full((len(rows),), -7.0, dtype=torch.float64, device="cuda")
    ctx.greedy(x, len(rows), V, ids, mg)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), mg.cpu().numpy()


def check(ctx, torch, rows):
    ids, mg = run(ctx, torch, rows)
    for r, row in enumerate(rows):
        want_id = host.argmax_first(list(np.asarray(row, np.float32)))
        want_mg = host.top_two_margin(list(np.asarray(row, np.float32)))
        assert int(ids[r]) == want_id, (r, row[:8], int(ids[r]), want_id)
        if math.isnan(want_mg):
            assert math.isnan(mg[r]), (r, mg[r])
        else:
            assert mg[r] == want_mg, (r, mg[r], want_mg)


def test_known_answers(ctx, torch_gpu):
    for c in GOLD["top_two_margin"]["cases"]:
        _, mg = run(ctx, torch_gpu, [c["logits"]])
        assert abs(mg[0] - c["want"]) <= 1e-6
    ids, _ = run(ctx, torch_gpu, [GOLD["argmax_ties"]["logits"]])
    assert ids[0] == GOLD["argmax_ties"]["want"]


@pytest.mark.parametrize("V", [2, 3, 5, 7, 8, 1023, 1024, 4099])
def test_crafted_rows(ctx, torch_gpu, V):
    rng = np.random.default_rng(V)
    base = lambda: list(rng.standard_normal(V).astype(np.float32))
    rows = []
    rows.append([1.0] * V)                                   # all equal: 0, margin 0
    rows.append([-inf] * V)                                  # all -inf: 0, margin NaN
    r = base(); r[0] = nan; rows.append(r)                   # NaN first: 0, NaN
    r = base(); r[-1] = nan; rows.append(r)                  # NaN last: never taken
    r = base(); r[1] = nan; r[0] = 100.0; rows.append(r)     # x[1] NaN, x[0] on top: NaN
    if V > 2:
        r = base(); r[1] = nan; r[V - 1] = 50.0; r[0] = 10.0; rows.append(r)  # displaced
        r = base(); m = max(r) + 1; r[V // 2] = m; r[V - 1] = m; rows.append(r)  # tie
        r = base(); r[V // 3] = inf; rows.append(r)           # +inf once
        r = base(); r[1] = inf; r[V - 1] = inf; rows.append(r)  # +inf twice: margin NaN
        r = base(); r[2] = nan; r[V - 2] = nan; rows.append(r)  # NaNs inside
    r = base(); r[0] = max(r) + 5; rows.append(r)             # max at index 0
    r = base(); rows.append([-x for x in r])
    check(ctx, torch_gpu, rows)


def test_vocabulary_rows_with_the_maximum_everywhere(ctx, torch_gpu):
    """V = 151936 over 16 workgroups per row (a thread's 16-byte chunks 1024 floats apart
    in its workgroup's chunk of the row): the maximum placed at both ends and inside,
    ties across threads, waves and workgroups resolved to the lowest index."""
    V = 151936
    rng = np.random.default_rng(1)
    rows = []
    for at in (0, 1, 3, 4, 4095, 4096, 4097, 65536 + 5, V - 5, V - 1):
        r = rng.standard_normal(V).astype(np.float32)
        r[at] = 9.0
        rows.append(r)
    r = rng.standard_normal(V).astype(np.float32)
    for at in (V - 1, 70000, 4100, 12):  # the same maximum four times
        r[at] = 9.0
    rows.append(r)
    r = rng.standard_normal(V).astype(np.float32)
    r[5000], r[140000] = 9.0, 9.0 - 2.0 ** -20  # a near tie: margin 2^-20 exactly
    rows.append(r)
    ids, mg = run(ctx, torch_gpu, rows)
    for i, row in enumerate(rows):
        assert int(ids[i]) == int(np.argmax(row))
        top = np.sort(row.astype(np.float64))[-2:]
        assert mg[i] == top[1] - top[0]
    assert ids[-2] == 12 and mg[-2] == 0.0
    assert mg[-1] == 2.0 ** -20


@pytest.mark.parametrize("V", [12291, 8192 + 4])
def test_rows_split_over_workgroups_at_any_offset(ctx, torch_gpu, V):
    """A few rows of V logits split over several workgroups each (V odd: element-wise
    chunks; V % 4 == 0: float4 chunks), with the maximum, its ties, NaNs and +inf placed
    around every possible chunk edge; against the Go loops."""
    rng = np.random.default_rng(V)
    rows = []
    for edge_frac in (1 / 3, 1 / 2, 2 / 3):
        e = int(V * edge_frac)
        for d in (-1, 0, 1):
            r = list(rng.standard_normal(V).astype(np.float32))
            r[e + d] = 11.0
            rows.append(r)
        r = list(rng.standard_normal(V).astype(np.float32))
        r[e - 1], r[e], r[e + 1] = 11.0, 11.0, float("nan")
        rows.append(r)
        r = list(rng.standard_normal(V).astype(np.float32))
        r[e + 1] = inf
        r[0] = nan
        rows.append(r)
    check(ctx, torch_gpu, rows)


@pytest.mark.parametrize("B", [1, 33, 100, 130, 600])
def test_batches_of_vocabulary_rows(ctx, torch_gpu, B):
    """B rows of 151936 logits (a row splits over up to 16 workgroups, fewer as B grows):
    per row the maximum repeated at random places (the first must win wherever the
    copies fall), a unique maximum, or a near tie; ids and margins against numpy's first
    argmax and the sorted top two."""
    torch = torch_gpu
    V = 151936
    rng = np.random.default_rng(B)
    x = rng.standard_normal((B, V)).astype(np.float32)
    for b in range(B):
        kind = b % 3
        if kind == 0:
            at = rng.choice(V, size=int(rng.integers(2, 9)), replace=False)
            x[b, at] = 7.5
        elif kind == 1:
            x[b, int(rng.integers(0, V))] = 8.0
        else:
            i, j = rng.choice(V, size=2, replace=False)
            x[b, i], x[b, j] = 6.0, 6.0 - 2.0 ** -18
    dx = torch.from_numpy(x).cuda()
    ids = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    mg = torch.full((B,), -7.0, dtype=torch.float64, device="cuda")
    ctx.greedy(dx, B, V, ids, mg)
    torch.cuda.synchronize()
    ids, mg = ids.cpu().numpy(), mg.cpu().numpy()
    top = np.partition(x, V - 2, axis=1)[:, -2:].astype(np.float64)
    assert np.array_equal(ids, np.argmax(x, axis=1))
    assert np.array_equal(mg, top[:, 1] - top[:, 0])
    assert np.array_equal(dx.cpu().numpy(), x)  # the logits are only read


def test_refusals(ctx, torch_gpu):
    import tgo_amd
    x = torch_gpu.zeros(4, device="cuda")
    ids = torch_gpu.zeros(4, dtype=torch_gpu.int32, device="cuda")
    with pytest.raises(tgo_amd.TgoError, match="at least two"):
        ctx.greedy(x, 4, 1, ids)
