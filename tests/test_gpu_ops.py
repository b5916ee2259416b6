"""GPU parity of the non-GEMM operators the reference's yolo26n chain needs:
max_pool2d_with_indices (values and int32 indices, ceil_mode, the chained
same-size pools of the SPPF block folded into one launch), permute_copy and
softmax, each against oracle/ops.py on the same seeded inputs.

Bars: max-pool values and indices and every permutation are bit-exact
(selection and index work); softmax is within
  float32  |y - y64| <= 1e-5 * sqrt(R) * y64 + 1e-30
  float16  |y - y64| <= 1e-2 * y64 + 1e-6   (subnormal outputs: 6e-8 spacing)
  bfloat16 |y - y64| <= 2e-2 * y64 + 1e-30
of the float64 softmax of the same (rounded) inputs, R the reduced extent.
"""
import numpy as np
import pytest

from gpu_util import round_in

pytestmark = pytest.mark.gpu

DTS = ["float32", "float16", "bfloat16"]


@pytest.fixture(scope="module")
def ctx(pkg):
    c = pkg.wgx.Context(0)
    yield c
    c.destroy()


def upload(ctx, a, dtype):
    return ctx.from_numpy(a.astype(np.float32), dtype)


# ------------------------------------------------------------------ max-pool
POOLS = [  # (shape, kernel, stride, padding, dilation, ceil_mode)
    ((1, 128, 20, 20), (5, 5), (1, 1), (2, 2), (1, 1), False),
    ((2, 3, 17, 23), (3, 3), (2, 2), (1, 1), (1, 1), False),
    ((2, 3, 17, 23), (3, 3), (2, 2), (1, 1), (1, 1), True),
    ((1, 4, 16, 15), (2, 3), (2, 1), (0, 1), (2, 1), False),
    ((1, 2, 9, 9), (4, 4), (3, 3), (1, 2), (1, 1), True),
    ((3, 5, 33, 65), (2, 2), (2, 2), (0, 0), (1, 1), False),
]


@pytest.mark.parametrize("dtype", DTS)
@pytest.mark.parametrize("geom", POOLS, ids=[f"{g[0][2]}x{g[0][3]}k{g[1][0]}{g[1][1]}s{g[2][0]}p{g[3][0]}{g[3][1]}d{g[4][0]}c{int(g[5])}" for g in POOLS])
def test_max_pool_values_and_indices(ctx, pkg, dtype, geom):
    from oracle import ops

    shape, k, s, p, d, ceil = geom
    I = pkg.inputs
    # integer-valued inputs in a small range: many ties, so the
    # first-strictly-greatest rule is exercised, not just the maximum
    a = np.floor(I.uniform(70, shape, -4, 4)).astype(np.float32)
    a = round_in(a, dtype)
    ref, ridx = ops.max_pool2d_with_indices(a, k, s, p, d, ceil, dtype)
    x = upload(ctx, a, dtype)
    y = ctx.tensor(dtype, list(ref.shape))
    ix = ctx.tensor("int32", list(ref.shape))
    print(f"[max_pool] {dtype} {geom}", flush=True)
    ctx.reset()
    ctx.max_pool2d(x, k, s, p, d, y, indices=ix, ceil_mode=ceil)
    ctx.submit()
    ctx.sync()
    np.testing.assert_array_equal(y.get_f32(), ref.astype(np.float32))
    np.testing.assert_array_equal(ix.get_data(), ridx)


@pytest.mark.parametrize("dtype", DTS)
def test_sppf_chain_with_indices_folds(ctx, pkg, dtype):
    """Three chained 5x5 same-size pools with indices (yolo26n's SPPF block:
    its three indices outputs share one memory region) fold into one launch;
    every level's values and the shared indices equal pooling step by step
    (the last level's indices stay, as after three launches)."""
    from oracle import ops

    I = pkg.inputs
    shape = (1, 128, 20, 20)
    a = round_in(np.floor(I.uniform(71, shape, -6, 6)).astype(np.float32), dtype)
    x = upload(ctx, a, dtype)
    ys = [ctx.tensor(dtype, list(shape)) for _ in range(3)]
    shared = ctx.tensor("int32", list(shape))
    args = ([5, 5], [1, 1], [2, 2], [1, 1])
    ctx.reset()
    for lvl, src in enumerate([x, ys[0], ys[1]]):
        ctx.max_pool2d(src, *args, ys[lvl], indices=shared)
    assert ctx.command_count == 1 and ctx.last_kernel == "max_pool2d_chain3"
    ctx.submit()
    ctx.sync()
    want = a
    for lvl in range(3):
        want, widx = ops.max_pool2d_with_indices(want, (5, 5), (1, 1), (2, 2), (1, 1), False, dtype)
        np.testing.assert_array_equal(ys[lvl].get_f32(), want.astype(np.float32))
    np.testing.assert_array_equal(shared.get_data(), widx)
    # distinct indices outputs per level fold too
    idx = [ctx.tensor("int32", list(shape)) for _ in range(3)]
    ctx.reset()
    for lvl, src in enumerate([x, ys[0], ys[1]]):
        ctx.max_pool2d(src, *args, ys[lvl], indices=idx[lvl])
    assert ctx.command_count == 1
    ctx.submit()
    ctx.sync()
    want = a
    for lvl in range(3):
        want, widx = ops.max_pool2d_with_indices(want, (5, 5), (1, 1), (2, 2), (1, 1), False, dtype)
        np.testing.assert_array_equal(idx[lvl].get_data(), widx)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_sppf_chain_does_not_fold_over_aliased_memory(ctx, pkg, dtype):
    """A pool whose output overlaps the chain's input (a memory plan may give
    y2 the space of the dead x) or an earlier output stays a launch of its
    own, and the results still equal pooling step by step."""
    from oracle import ops

    I = pkg.inputs
    shape = (1, 8, 12, 12)
    n = int(np.prod(shape))
    a = round_in(I.uniform(72, shape, -3, 3), dtype)
    args = ([5, 5], [1, 1], [2, 2], [1, 1])
    buf = ctx.storage_buffer(3 * n * 2)
    x = ctx.tensor(dtype, list(shape), buffer=buf)
    y1 = ctx.tensor(dtype, list(shape), buffer=buf + n * 2)
    y3 = ctx.tensor(dtype, list(shape), buffer=buf + 2 * n * 2)
    # y2 takes x's memory: the second pool must run after the first as a launch of its own
    ctx.reset()
    x.set_data(np.asarray(pkg.wgx.f32_to_bf16_bits(a) if dtype == "bfloat16" else a.astype(np.float16)))
    ctx.max_pool2d(x, *args, y1)
    ctx.max_pool2d(y1, *args, x)
    assert ctx.command_count == 2
    ctx.max_pool2d(x, *args, y3)  # pools the previous output again: may join the second launch
    ctx.submit()
    ctx.sync()
    w1, _ = ops.max_pool2d_with_indices(a, (5, 5), (1, 1), (2, 2), (1, 1), False, dtype)
    w2, _ = ops.max_pool2d_with_indices(w1, (5, 5), (1, 1), (2, 2), (1, 1), False, dtype)
    w3, _ = ops.max_pool2d_with_indices(w2, (5, 5), (1, 1), (2, 2), (1, 1), False, dtype)
    np.testing.assert_array_equal(y1.get_f32(), w1.astype(np.float32))
    np.testing.assert_array_equal(x.get_f32(), w2.astype(np.float32))
    np.testing.assert_array_equal(y3.get_f32(), w3.astype(np.float32))
    # y2 overlapping y1 (not x): also separate
    ctx.reset()
    z = [ctx.tensor(dtype, list(shape)) for _ in range(2)]
    x2 = upload(ctx, a, dtype)
    ctx.max_pool2d(x2, *args, z[0])
    ctx.max_pool2d(z[0], *args, z[0])
    assert ctx.command_count == 2
    ctx.submit()
    ctx.sync()
    # pooling in place: the result depends on the order of the in-place
    # writes, which neither the reference nor this library defines; only
    # the launch count is the contract here


# ------------------------------------------------------------------ permute
PERMS = [((2, 3), (1, 0)), ((1, 2, 400, 400), (0, 1, 3, 2)), ((1, 2, 32, 400), (0, 1, 3, 2)),
         ((3, 70, 129), (0, 2, 1)), ((2, 3, 4, 5), (3, 1, 0, 2)), ((5, 1, 7, 2, 3), (4, 2, 0, 3, 1)),
         ((64, 48), (-1, 0)), ((1,), (0,))]


@pytest.mark.parametrize("dtype", DTS)
@pytest.mark.parametrize("shape,dims", PERMS, ids=[f"{'x'.join(map(str, s))}_{''.join(map(str, d))}" for s, d in PERMS])
def test_permute_is_exact(ctx, pkg, dtype, shape, dims):
    from oracle import ops

    a = round_in(pkg.inputs.normal(73, shape), dtype)
    want = ops.permute(a, dims)
    x = upload(ctx, a, dtype)
    y = ctx.tensor(dtype, list(want.shape))
    ctx.reset()
    ctx.permute(x, dims, y)
    ctx.submit()
    ctx.sync()
    np.testing.assert_array_equal(y.get_f32(), want)


# ------------------------------------------------------------------ softmax
SOFTMAX = [((1, 2, 400, 400), -1), ((2, 3), 1), ((2, 2), 0), ((4, 1000), 1), ((3, 7, 5), 1),
           ((2, 8400), 0), ((1, 84, 8400), 2), ((5, 3, 2), 0), ((16, 64), -1)]


@pytest.mark.parametrize("dtype", DTS)
@pytest.mark.parametrize("shape,dim", SOFTMAX, ids=[f"{'x'.join(map(str, s))}_d{d}" for s, d in SOFTMAX])
def test_softmax_parity(ctx, pkg, dtype, shape, dim):
    from oracle import ops

    a = round_in(pkg.inputs.normal(74, shape, 0.0, 3.0), dtype)
    want = ops.softmax_f64(a, dim)
    R = shape[dim]
    x = upload(ctx, a, dtype)
    y = ctx.tensor(dtype, list(shape))
    ctx.reset()
    ctx.softmax(x, dim, y)
    ctx.submit()
    ctx.sync()
    got = y.get_f32().astype(np.float64)
    if dtype == "float32":
        bound = 1e-5 * np.sqrt(R) * want + 1e-30
    elif dtype == "float16":
        bound = 1e-2 * want + 1e-6
    else:
        bound = 2e-2 * want + 1e-30
    err = np.abs(got - want)
    assert np.all(err <= bound), f"{int((err > bound).sum())} outside; worst {np.max(err / bound):.3g} of the bound"


def test_softmax_in_place(ctx, pkg):
    from oracle import ops

    a = pkg.inputs.normal(75, (8, 333))
    want = ops.softmax_f64(a, 1)
    x = upload(ctx, a, "float32")
    ctx.reset()
    ctx.softmax(x, 1, x)
    ctx.submit()
    ctx.sync()
    np.testing.assert_allclose(x.get_f32(), want, rtol=1e-5 * np.sqrt(333), atol=1e-30)
