"""nn.Linear on the GPU (every weight form) against the CPU restatement.

Dequantization is bit-exact: the device's f32 dequant equals the host
restatement's, and the f16 operand of the f16-activation path equals the
round-to-nearest-even f16 of that value. With f32 activations (tgo's
arithmetic) the product multiplies the unrounded dequantized weight (carried as
two f16 parts whose sum is exact) by the activation carried as f16 hi + lo.
The product is compared with a float64 matmul of exactly those operands -- the
f16-rounded weights and activations on the f16 path, the f32 dequantized
weights and f32 activations on the f32 path -- so the budget is f32
accumulation, written here as in tolerance.go:
    |y - y_ref| <= 4 * sqrt(K) * 2^-24 * sum_k |x_k w_k|      (AccumF32(K), headroom 4)
plus, on the f32 path, the activation's low part's own rounding: 2^-22 * sum |x_k w_k|.
That is the budget of the reference's own quantized-matmul parity test
(internal/conformance/parity_test.go:233-281: accel's QuantMatMul against a
float64 matmul of the dequantized weights, AccumF32 only). Against tgo's CPU
path (f32 activations, the same dequantized weights) the f16 path's budget adds
the f16 operand term StoreF16, 2^-11 per rounded operand.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

FORMS = {0: "f16", 1: "int8", 2: "int4-tgo", 3: "int4-sym"}


def make_weight(form, K, N, rng):
    w = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    if form == 0:
        return dict(plane=oracle.f16_bits(w)), None
    if form == 1:
        q = np.empty(K * N, np.int8)
        s = np.empty((K * N + 31) // 32, np.uint16)
        oracle.lib.orc_quantize_int8(oracle.ptr(w.ravel().copy()), K * N, oracle.ptr(q), oracle.ptr(s))
        return dict(plane=q, scales=s), None
    if form == 2:
        c = np.empty((K * N + 7) // 8, np.uint32)
        s = np.empty((K * N + 127) // 128, np.uint16)
        z = np.empty((K * N + 127) // 128, np.uint16)
        oracle.lib.orc_quantize_int4_tgo(oracle.ptr(w.ravel().copy()), K * N, oracle.ptr(c),
                                         oracle.ptr(s), oracle.ptr(z))
        return dict(plane=c, scales=s, zeros=z), None
    qw, sc = oracle.synth_int4_sym(7, 3, K, N, 0.01)
    return dict(plane=qw, scales=sc), None


def deq(form, K, N, wd):
    return oracle.dequant(form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))


@pytest.mark.parametrize("form", [0, 1, 2, 3])
def test_dequant_is_bit_exact(ctx, torch_gpu, form):
    torch = torch_gpu
    rng = np.random.default_rng(form)
    K, N = 256, 384
    wd, _ = make_weight(form, K, N, rng)
    h = ctx.weight_upload(form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))
    try:
        y = torch.empty((K, N), dtype=torch.float32, device="cuda")
        ctx.dequant(h, y)
        y16 = torch.empty((K, N), dtype=torch.float16, device="cuda")
        ctx.dequant_f16(h, y16)
        torch.cuda.synchronize()
        want = deq(form, K, N, wd)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
        assert np.array_equal(y16.cpu().numpy().view(np.uint16),
                              want.astype(np.float16).view(np.uint16))
    finally:
        ctx.weight_free(h)


def split_pair(x):
    """An f32 activation as tgo's arithmetic carries it: f16 hi, then f16 lo = f16(x - hi)."""
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


@pytest.mark.parametrize("form", [0, 1, 2, 3])
@pytest.mark.parametrize("M", [1, 8, 16, 32, 33, 64, 130, 300])
@pytest.mark.parametrize("xk", ["f32", "f16", "x2"])
def test_linear_matches_the_oracle(ctx, torch_gpu, form, M, xk):
    """xk: f32 activations (split in the kernel), f16, or an activation pair (f16 hi plane
    then lo plane, the form precision mode 1's producers write; the exact pipelined kernel
    from 33 rows)."""
    torch = torch_gpu
    import tgo_amd
    xf32 = xk != "f16"
    rng = np.random.default_rng(100 + form * 7 + M)
    K, N = 512, 256 if form != 2 else 384
    wd, _ = make_weight(form, K, N, rng)
    w32 = deq(form, K, N, wd)
    w16 = w32.astype(np.float16).astype(np.float64)
    x = rng.standard_normal((M, K)).astype(np.float32)
    h = ctx.weight_upload(form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))
    try:
        if xk == "f32":
            dx = torch.from_numpy(x).cuda()
            xu = x.astype(np.float64)
        elif xk == "x2":
            hi, lo = split_pair(x)
            dx = torch.from_numpy(np.concatenate([hi.ravel(), lo.ravel()])).cuda()
            xu = x.astype(np.float64)
        else:
            dx = torch.from_numpy(x.astype(np.float16)).cuda()
            xu = x.astype(np.float16).astype(np.float64)
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        ctx.linear(h, dx, M, y, x_dtype={"f32": tgo_amd.F32, "f16": tgo_amd.F16,
                                         "x2": tgo_amd.F16X2}[xk])
        torch.cuda.synchronize()
        got = y.cpu().numpy().astype(np.float64)
    finally:
        ctx.weight_free(h)
    wop = w32.astype(np.float64) if xf32 else w16  # the weights the product multiplies
    ref = xu @ wop
    mag = np.abs(xu) @ np.abs(wop)
    tol = (4 * np.sqrt(K) * 2.0 ** -24 + (2.0 ** -22 if xf32 else 0)) * mag + 1e-30
    assert np.all(np.abs(got - ref) <= tol), np.max(np.abs(got - ref) / tol)
    # against tgo's CPU path (f32 activations, unrounded f32 weights)
    cpu = oracle.cpu_linear(x, form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))
    mag2 = np.abs(x.astype(np.float64)) @ np.abs(w32.astype(np.float64))
    tol2 = ((2.0 ** -22 if xf32 else 2 * 2.0 ** -11) + 8 * np.sqrt(K) * 2.0 ** -24) * mag2
    assert np.all(np.abs(got - cpu) <= tol2), np.max(np.abs(got - cpu) / tol2)


@pytest.mark.parametrize("K", [512, 2048])
@pytest.mark.parametrize("M", [64, 200])
def test_exact_int4_sym_scales_across_the_f16_range(ctx, torch_gpu, K, M):
    """Symmetric int4 in tgo's arithmetic (activation pairs, the pipelined exact kernel:
    K = 512 one unsplit launch with two k groups per workgroup, K = 2048 split-K) with
    group scales planted across f16's whole range: the largest finite (65504, so
    |q s| reaches 524032, past f16), large, ordinary, the smallest normal and
    subnormal. The kernel multiplies the exact codes and applies each group's scale in
    f32, so every product stays the f32 dequantized weight's; against the f64 product
    of the f32 activations and the oracle's dequantization, AccumF32 + 2^-22."""
    torch = torch_gpu
    import tgo_amd
    N = 256
    qw, sc = oracle.synth_int4_sym(11, 4, K, N, 0.02)
    planted = np.array([65504.0, 60000.0, 1000.0, 1.0, 0.01, 2.0 ** -14, 2.0 ** -20, 2.0 ** -24],
                       np.float16).view(np.uint16)
    g = np.arange(K // 32)[:, None] + 3 * np.arange(N)[None, :]
    sc = np.ascontiguousarray(planted[g % len(planted)])
    w64 = oracle.dequant(3, K, N, qw, sc).astype(np.float64)
    assert np.isfinite(w64).all() and np.abs(w64).max() > 65504
    rng = np.random.default_rng(K + M)
    x = rng.standard_normal((M, K)).astype(np.float32)
    hi, lo = split_pair(x)
    h = ctx.weight_upload(3, K, N, qw, sc)
    try:
        dx = torch.from_numpy(np.concatenate([hi.ravel(), lo.ravel()])).cuda()
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        ctx.linear(h, dx, M, y, x_dtype=tgo_amd.F16X2)
        torch.cuda.synchronize()
        got = y.cpu().numpy().astype(np.float64)
    finally:
        ctx.weight_free(h)
    xu = x.astype(np.float64)
    ref = xu @ w64
    tol = (4 * np.sqrt(K) * 2.0 ** -24 + 2.0 ** -22) * (np.abs(xu) @ np.abs(w64))
    assert np.all(np.abs(got - ref) <= tol), np.max(np.abs(got - ref) / tol)


def test_linear_is_deterministic_and_row_independent(ctx, torch_gpu):
    """A row's result does not depend on the rows beside it when the tile
    configuration is the same (M in one tile class)."""
    torch = torch_gpu
    import tgo_amd
    rng = np.random.default_rng(3)
    K, N = 1024, 512
    qw, sc = oracle.synth_int4_sym(1, 9, K, N, 0.01)
    h = ctx.weight_upload(3, K, N, qw, sc)
    try:
        x = torch.randn(200, K, device="cuda").half()
        y1 = torch.empty(200, N, device="cuda")
        y2 = torch.empty(200, N, device="cuda")
        ctx.linear(h, x, 200, y1, x_dtype=tgo_amd.F16)
        ctx.linear(h, x, 200, y2, x_dtype=tgo_amd.F16)
        x2 = x.clone()
        x2[150:] = 0
        y3 = torch.empty(200, N, device="cuda")
        ctx.linear(h, x2, 200, y3, x_dtype=tgo_amd.F16)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)
        assert torch.equal(y1[:128], y3[:128])
    finally:
        ctx.weight_free(h)


def sym_codes_and_columns(K, N, seed, stream, sigma, cols):
    """Host int4-sym codes (the oracle's seeded generator) and the oracle's f32
    dequantization of the sampled columns: the codes go up through the product's
    upload and repack, the reference never touches the device's weights."""
    qw, sc = oracle.synth_int4_sym(seed, stream, K, N, sigma)
    wc = oracle.dequant(3, K, len(cols), np.ascontiguousarray(qw[:, cols]),
                        np.ascontiguousarray(sc[:, cols]))
    return qw, sc, wc


@pytest.mark.parametrize("KN", [(4096, 12288), (12288, 4096), (4096, 6144)])
def test_c3_shapes_sampled_columns(ctx, torch_gpu, KN):
    """BASELINE config 3 shapes (int4 symmetric, group 32 along K) at M = 1..1024,
    checked on sampled columns against the f64 product of the same f16 operands, the
    weights dequantized by the oracle from the host's codes."""
    torch = torch_gpu
    import tgo_amd
    K, N = KN
    cols = np.arange(0, N, N // 64)
    qw, sc, wc = sym_codes_and_columns(K, N, 42, 5, 0.02, cols)
    w16 = torch.from_numpy(wc.astype(np.float16).astype(np.float64)).cuda()
    h = ctx.weight_upload(3, K, N, qw, sc)
    try:
        dcols = torch.from_numpy(cols).cuda()
        for M in (1, 8, 64, 256, 1024):
            x = torch.randn(M, K, device="cuda").half()
            y = torch.empty(M, N, device="cuda")
            ctx.linear(h, x, M, y, x_dtype=tgo_amd.F16)
            torch.cuda.synchronize()
            ref = x.double() @ w16
            mag = x.double().abs() @ w16.abs()
            tol = 4 * (K ** 0.5) * 2.0 ** -24 * mag
            assert bool(((y[:, dcols].double() - ref).abs() <= tol).all()), M
    finally:
        ctx.weight_free(h)


@pytest.mark.parametrize("KN", [(4096, 12288), (12288, 4096), (4096, 6144), (4096, 24576)])
def test_c3_shapes_tgo_arithmetic_sampled_columns(ctx, torch_gpu, KN):
    """The same shapes in tgo's arithmetic (activation pairs, the exact kernel) at the
    step's row counts, against the f64 product of the f32 activations and the oracle's
    f32 dequantized weights, AccumF32 + 2^-22; [4096, 24576] is the fused gate/up."""
    torch = torch_gpu
    import tgo_amd
    K, N = KN
    cols = np.arange(0, N, N // 64)
    qw, sc, wc = sym_codes_and_columns(K, N, 43, 6, 0.02, cols)
    w64 = torch.from_numpy(wc.astype(np.float64)).cuda()
    h = ctx.weight_upload(3, K, N, qw, sc)
    try:
        dcols = torch.from_numpy(cols).cuda()
        for M in (128, 1152, 1280):
            x = torch.randn(M, K, device="cuda")
            hi = x.half()
            lo = (x - hi.float()).half()
            xp = torch.cat([hi.reshape(-1), lo.reshape(-1)])
            y = torch.empty(M, N, device="cuda")
            ctx.linear(h, xp, M, y, x_dtype=tgo_amd.F16X2)
            torch.cuda.synchronize()
            ref = x.double() @ w64
            mag = x.double().abs() @ w64.abs()
            tol = (4 * (K ** 0.5) * 2.0 ** -24 + 2.0 ** -22) * mag
            assert bool(((y[:, dcols].double() - ref).abs() <= tol).all()), M
    finally:
        ctx.weight_free(h)


@pytest.mark.parametrize("form", [0, 1, 2, 3])
@pytest.mark.parametrize("M", [1, 5, 8, 9, 32])
def test_small_m_forms_against_the_oracle(ctx, torch_gpu, form, M):
    """Every weight form through the small-M kernels at K = 2048 (the staged form at 1-8
    rows, direct at 9-32), f16 activations, against the float64 product of the same
    operands and against tgo's CPU path (f32 activations, unrounded weights)."""
    torch = torch_gpu
    import tgo_amd
    rng = np.random.default_rng(500 + form * 11 + M)
    K, N = 2048, 512 if form != 2 else 640
    wd, _ = make_weight(form, K, N, rng)
    w32 = deq(form, K, N, wd)
    w16 = w32.astype(np.float16).astype(np.float64)
    x = rng.standard_normal((M, K)).astype(np.float32)
    h = ctx.weight_upload(form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))
    try:
        dx = torch.from_numpy(x.astype(np.float16)).cuda()
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        ctx.linear(h, dx, M, y, x_dtype=tgo_amd.F16)
        torch.cuda.synchronize()
        got = y.cpu().numpy().astype(np.float64)
    finally:
        ctx.weight_free(h)
    xu = x.astype(np.float16).astype(np.float64)
    ref = xu @ w16
    mag = np.abs(xu) @ np.abs(w16)
    tol = 4 * np.sqrt(K) * 2.0 ** -24 * mag + 1e-30
    assert np.all(np.abs(got - ref) <= tol), np.max(np.abs(got - ref) / tol)
    cpu = oracle.cpu_linear(x, form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))
    mag2 = np.abs(x.astype(np.float64)) @ np.abs(w32.astype(np.float64))
    tol2 = (2.0 ** -11 * 2 + 8 * np.sqrt(K) * 2.0 ** -24) * mag2
    assert np.all(np.abs(got - cpu) <= tol2)


@pytest.mark.parametrize("KN", [(4096, 6144), (12288, 4096), (4096, 24576), (4096, 151936)])
def test_small_m_kernel_against_its_operands(ctx, torch_gpu, KN):
    """The small-M kernels (at most 32 rows; 1-8 rows on the 16x16x32 pairing) at the
    8B projection shapes, 16 waves per column block (QKV [4096, 6144], down [12288, 4096])
    and 4 (gate/up [4096, 24576], LM head [4096, 151936]): f32 output on sampled columns
    against the f64 product of the same operands (the weights dequantized by the oracle
    from the host's codes); repeated calls bit-equal; the f16 output is the f16 rounding of
    the same sums."""
    torch = torch_gpu
    import tgo_amd
    K, N = KN
    ncols = np.arange(0, N, max(1, N // 96))
    qw, sc, wcols = sym_codes_and_columns(K, N, 11, 5, 0.02, ncols)
    h = ctx.weight_upload(3, K, N, qw, sc)
    del qw, sc
    try:
        cols = torch.from_numpy(ncols).cuda()
        wc = torch.from_numpy(wcols.astype(np.float16).astype(np.float64)).cuda()
        for M in (1, 3, 8, 9, 32):
            print("small-M linear [%d,%d] M=%d" % (K, N, M), flush=True)
            x = torch.randn(M, K, device="cuda").half()
            ys = []
            for _ in range(3):
                y = torch.full((M, N), float("nan"), device="cuda")
                ctx.linear(h, x, M, y, x_dtype=tgo_amd.F16)
                ys.append(y)
            y16 = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
            ctx.linear(h, x, M, y16, x_dtype=tgo_amd.F16, y_dtype=tgo_amd.F16)
            torch.cuda.synchronize()
            assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2]), M
            assert torch.equal(y16, ys[0].half()), M
            ref = x.double() @ wc
            mag = x.double().abs() @ wc.abs()
            tol = 4 * (K ** 0.5) * 2.0 ** -24 * mag
            assert bool(((ys[0][:, cols].double() - ref).abs() <= tol).all()), M
    finally:
        ctx.weight_free(h)


@pytest.mark.parametrize("M", [33, 131, 1152])
@pytest.mark.parametrize("KN", [(2048, 416), (512, 3712)])
@pytest.mark.parametrize("form", [3, 2, 1])
def test_large_m_exact_ragged_edges(ctx, torch_gpu, M, KN, form):
    """The pipelined exact path (activation pairs, tgo's arithmetic; symmetric int4 with its
    group scale applied in f32, the other forms with the exact weight pair) at partial row
    and column tiles: N = 416 and 3712 leave the last 256-column tile 160 and 128 columns
    wide; K = 2048 at 33 and 131 rows splits K. Every column against the f64 product of the
    f32 activations and the oracle's f32 dequantized weights, AccumF32 + 2^-22."""
    torch = torch_gpu
    import tgo_amd
    K, N = KN
    if form == 2 and N % 128:
        N = 512  # tgo's int4 groups run along N in 128s
    wd, _ = make_weight(form, K, N, np.random.default_rng(29 + M))
    w64 = torch.from_numpy(deq(form, K, N, wd).astype(np.float64)).cuda()
    h = ctx.weight_upload(form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))
    try:
        x = torch.randn(M, K, device="cuda")
        hi = x.half()
        lo = (x - hi.float()).half()
        y = torch.full((M, N), float("nan"), device="cuda")
        ctx.linear(h, torch.cat([hi.reshape(-1), lo.reshape(-1)]), M, y, x_dtype=tgo_amd.F16X2)
        torch.cuda.synchronize()
        ref = x.double() @ w64
        tol = (4 * (K ** 0.5) * 2.0 ** -24 + 2.0 ** -22) * (x.double().abs() @ w64.abs())
        assert bool(((y.double() - ref).abs() <= tol).all())
    finally:
        ctx.weight_free(h)


@pytest.mark.parametrize("M", [33, 47, 96, 131, 300, 1000, 1152])
@pytest.mark.parametrize("KN", [(2048, 416), (512, 4096), (512, 3712)])
@pytest.mark.parametrize("form", [3, 2, 1])
def test_large_m_tiles_ragged_edges(ctx, torch_gpu, M, KN, form):
    """The pipelined f16-activation path at M >= 33 (64- and 128-row tiles, 4
    or 8 waves wide, XCD-dealt, split-K when the tiles alone do not fill the
    chip; int8 and tgo's int4 with their scales through LDS): partial row and
    column tiles and every column checked against the f64 product of the same
    f16 operands. N = 4096 and 3712 (116 column blocks: the last 512-column
    tile holds 4) run 128-row tiles 8 waves wide. The weights are the host's codes, the
    reference's dequantized by the oracle."""
    torch = torch_gpu
    import tgo_amd
    K, N = KN
    if form == 2 and N % 128:
        N = 512  # tgo's int4 groups run along N in 128s
    wd, _ = make_weight(form, K, N, np.random.default_rng(17 + M))
    wf = torch.from_numpy(deq(form, K, N, wd).astype(np.float16)).cuda()
    h = ctx.weight_upload(form, K, N, wd["plane"], wd.get("scales"), wd.get("zeros"))
    try:
        x = torch.randn(M, K, device="cuda").half()
        y = torch.full((M, N), float("nan"), device="cuda")
        ctx.linear(h, x, M, y, x_dtype=tgo_amd.F16)
        y16 = torch.full((M, N), float("nan"), device="cuda", dtype=torch.float16)
        ctx.linear(h, x, M, y16, x_dtype=tgo_amd.F16, y_dtype=tgo_amd.F16)
        torch.cuda.synchronize()
        ref = x.double() @ wf.double()
        mag = x.double().abs() @ wf.double().abs()
        tol = 4 * (K ** 0.5) * 2.0 ** -24 * mag
        assert bool(((y.double() - ref).abs() <= tol).all())
        assert torch.equal(y16, y.half())
    finally:
        ctx.weight_free(h)
