"""GPU tests of the execution model: submit/sync/reset semantics, copies,
setData prefixes and graph replays (src/context.ts:172-389, src/tensor.ts:115-158).
"""
import numpy as np
import pytest

from gpu_util import assert_parity

pytestmark = pytest.mark.gpu


def test_copy_and_prefix_write(pkg):
    W = pkg.wgx
    ctx = W.Context(0)
    try:
        src = ctx.tensor("float32", [4]).set_data(np.array([1, 2, 3, 4], np.float32))
        dst = ctx.tensor("float32", [4])
        ctx.copy(src, dst)
        ctx.submit()
        ctx.sync()
        assert dst.get_data().tolist() == [1, 2, 3, 4]
        t = ctx.tensor("float32", [2, 3]).set_data(np.arange(1, 7, dtype=np.float32))
        t.set_data(np.array([7, 8], np.float32))
        assert t.get_data().ravel().tolist() == [7, 8, 3, 4, 5, 6]
        u = ctx.tensor("uint8", [3]).set_data(np.array([7, 42, 99], np.uint8))
        assert u.get_data().tolist() == [7, 42, 99]
        ctx.reset()
        ctx.submit()  # empty: no-op
        ctx.sync()
    finally:
        ctx.destroy()


def test_graph_replays_match_eager(pkg, orc):
    """Every replay of the captured graph equals the eager launch sequence,
    with eager work and synchronisations between the replays."""
    W, I = pkg.wgx, pkg.inputs
    results = {}
    for graph in (False, True):
        ctx = W.Context(0)
        try:
            ctx.set_graph_mode(graph)
            x = I.as_f16(I.uniform(1, (1, 32, 24, 24), -1, 1))
            w1 = I.as_f16(I.kaiming_uniform(2, (64, 32, 3, 3)))
            w2 = I.as_f16(I.uniform(3, (64, 1, 3, 3), -0.5, 0.5))
            tx, t1, t2 = (ctx.from_numpy(a, "float16") for a in (x, w1, w2))
            y1 = ctx.tensor("float16", [1, 64, 24, 24])
            y2 = ctx.tensor("float16", [1, 64, 24, 24])
            y3 = ctx.tensor("float16", [1, 64, 24, 24])
            ctx.convolution(tx, t1, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 1, y1)
            ctx.unary("sigmoid", y1, y2)
            ctx.mul(y1, y2, y2)
            ctx.convolution(y2, t2, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 64, y3)
            outs = []
            for rep in range(4):
                ctx.submit()
                ctx.sync()
                outs.append(y3.get_data().copy())
                # eager work in between: overwrite the intermediate, then replay again
                y1.set_data(np.zeros((1, 64, 24, 24), np.float16))
            for o in outs[1:]:
                assert np.array_equal(o.view(np.uint16), outs[0].view(np.uint16))
            results[graph] = outs[0]
        finally:
            ctx.destroy()
    assert np.array_equal(results[True].view(np.uint16), results[False].view(np.uint16))


def test_graph_keeps_buffer_order(pkg):
    """A captured graph of independent and dependent commands (two unrelated
    convolutions and an mm, an add joining two of them, a read after write
    through a copy, an overwrite of an input an earlier command read): each
    replay equals the eager sequence bit for bit, replay after replay."""
    W, I = pkg.wgx, pkg.inputs
    results = {}
    for graph in (False, True):
        ctx = W.Context(0)
        try:
            ctx.set_graph_mode(graph)
            xa = ctx.from_numpy(I.as_f16(I.uniform(1, (1, 32, 40, 40), -1, 1)), "float16")
            wa = ctx.from_numpy(I.as_f16(I.kaiming_uniform(2, (64, 32, 3, 3))), "float16")
            xb = ctx.from_numpy(I.as_f16(I.uniform(3, (1, 64, 40, 40), -1, 1)), "float16")
            wb = ctx.from_numpy(I.as_f16(I.kaiming_uniform(4, (64, 64, 1, 1))), "float16")
            ma = ctx.from_numpy(I.as_f16(I.uniform(5, (512, 256), -1, 1)), "float16")
            mb = ctx.from_numpy(I.as_f16(I.uniform(6, (256, 384), -1, 1)), "float16")
            xnew = ctx.from_numpy(I.as_f16(I.uniform(7, (1, 32, 40, 40), -1, 1)), "float16")
            wz = ctx.from_numpy(I.as_f16(I.uniform(8, (64, 1, 3, 3), -0.5, 0.5)), "float16")
            ya, yb, s_, z, yz = (ctx.tensor("float16", [1, 64, 40, 40]) for _ in range(5))
            yc = ctx.tensor("float16", [512, 384])
            ctx.convolution(xa, wa, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 1, ya)
            ctx.convolution(xb, wb, None, [1, 1], [0, 0], [1, 1], False, [0, 0], 1, yb)   # independent
            ctx.mm(ma, mb, yc)                                                            # independent
            ctx.add(ya, yb, s_)                                                           # joins both
            ctx.copy(s_, z)                                                               # read after write
            ctx.convolution(z, wz, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 64, yz)
            ctx.copy(xnew, xa)                                   # overwrites an input the first conv read
            outs = []
            for rep in range(3):
                ctx.submit()
                ctx.sync()
                outs.append([t.get_data().copy() for t in (ya, yb, yc, s_, z, yz, xa)])
            results[graph] = outs
        finally:
            ctx.destroy()
    for rep, (e, g) in enumerate(zip(results[False], results[True])):
        for k, (a, b) in enumerate(zip(e, g)):
            assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"replay {rep} tensor {k}"
    # the second replay's first conv read the overwritten input
    assert not np.array_equal(results[True][0][0].view(np.uint16), results[True][1][0].view(np.uint16))


def test_time_submits_positive(pkg):
    W, I = pkg.wgx, pkg.inputs
    ctx = W.Context(0)
    try:
        a = ctx.from_numpy(I.uniform(1, (256, 256), -1, 1), "float16")
        b = ctx.from_numpy(I.uniform(2, (256, 256), -1, 1), "float16")
        o = ctx.tensor("float16", [256, 256])
        ctx.mm(a, b, o)
        ms = ctx.time_submits(10)
        assert 0.0 < ms < 100.0
    finally:
        ctx.destroy()


def test_elementwise_ops(pkg, orc):
    W, I = pkg.wgx, pkg.inputs
    ctx = W.Context(0)
    try:
        a = I.as_f16(I.uniform(10, (2, 3, 4, 5), -3, 3))
        b = I.as_f16(I.uniform(11, (1, 3, 1, 5), -3, 3))
        ta, tb = ctx.from_numpy(a, "float16"), ctx.from_numpy(b, "float16")
        o_add, o_mul, o_sig = (ctx.tensor("float16", [2, 3, 4, 5]) for _ in range(3))
        ctx.add(ta, tb, o_add, alpha=2.0)
        ctx.mul(ta, tb, o_mul)
        ctx.unary("sigmoid", ta, o_sig)
        c1 = ctx.tensor("float16", [2, 3, 4, 5])
        c2 = ctx.tensor("float16", [2, 2, 4, 5])
        cat = ctx.tensor("float16", [2, 5, 4, 5])
        ctx.copy(o_add, c1)
        ctx.split(ta, 1, [ctx.tensor("float16", [2, 1, 4, 5]), c2])
        ctx.cat([c1, c2], 1, cat)
        up = ctx.tensor("float16", [2, 3, 8, 10])
        ctx.upsample_nearest2d(ta, up)
        mp = ctx.tensor("float16", [2, 3, 4, 5])
        ctx.max_pool2d(ta, [5, 5], [1, 1], [2, 2], [1, 1], mp)
        ctx.submit()
        ctx.sync()
        ad = a.astype(np.float64)
        bd = b.astype(np.float64)
        np.testing.assert_allclose(o_add.get_f32(), ad + 2 * bd, atol=1e-2)
        np.testing.assert_allclose(o_mul.get_f32(), ad * bd, rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(o_sig.get_f32(), 1 / (1 + np.exp(-ad)), atol=2e-3)
        np.testing.assert_allclose(cat.get_f32(), np.concatenate([o_add.get_f32(), a[:, 1:]], 1))
        np.testing.assert_array_equal(up.get_f32(), a.repeat(2, 2).repeat(2, 3))
        pad = np.pad(ad, ((0, 0), (0, 0), (2, 2), (2, 2)), constant_values=-np.inf)
        ref = np.max(np.stack([pad[:, :, i:i + 4, j:j + 5] for i in range(5) for j in range(5)]), 0)
        np.testing.assert_array_equal(mp.get_f32(), ref)
    finally:
        ctx.destroy()


def _np_maxpool_same(a, k):
    p = k // 2
    pad = np.pad(a.astype(np.float64), ((0, 0), (0, 0), (p, p), (p, p)), constant_values=-np.inf)
    H, W = a.shape[2], a.shape[3]
    return np.max(np.stack([pad[:, :, i:i + H, j:j + W] for i in range(k) for j in range(k)]), 0)


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_chained_max_pools_fold(pkg, dtype):
    """Consecutive same-size max-pools, each pooling the previous output (the
    SPPF block), fold into one launch that writes every output; the results
    equal pooling step by step.  A pool whose input is not the previous
    output, or whose output overlaps the chain's input, stays separate."""
    W, I = pkg.wgx, pkg.inputs
    ctx = W.Context(0)
    try:
        a = I.uniform(40, (2, 8, 13, 17), -3, 3).astype(np.float16 if dtype == "float16" else np.float32)
        x = ctx.from_numpy(a, dtype)
        ys = [ctx.tensor(dtype, [2, 8, 13, 17]) for _ in range(4)]
        args = ([5, 5], [1, 1], [2, 2], [1, 1])
        ctx.max_pool2d(x, *args, ys[0])
        ctx.max_pool2d(ys[0], *args, ys[1])
        assert ctx.last_kernel == "max_pool2d_chain2"
        ctx.max_pool2d(ys[1], *args, ys[2])
        assert ctx.last_kernel == "max_pool2d_chain3"
        n_cmds = ctx.command_count
        ctx.max_pool2d(ys[2], *args, ys[3])  # a fourth does not join (at most 3)
        assert ctx.command_count == n_cmds + 1
        ctx.submit()
        ctx.sync()
        want = a.astype(np.float64)
        for y in ys:
            want = _np_maxpool_same(want, 5)
            np.testing.assert_array_equal(y.get_f32(), want.astype(np.float32))
        # no fold: the second pool reads the chain's input, not its output
        ctx.reset()
        z = [ctx.tensor(dtype, [2, 8, 13, 17]) for _ in range(2)]
        ctx.max_pool2d(x, *args, z[0])
        ctx.max_pool2d(x, [3, 3], [1, 1], [1, 1], [1, 1], z[1])
        assert ctx.command_count == 2
        ctx.submit()
        ctx.sync()
        np.testing.assert_array_equal(z[1].get_f32(), _np_maxpool_same(a, 3).astype(np.float32))
    finally:
        ctx.destroy()


def test_shared_contexts_order_and_freed_buffers(pkg):
    """Two contexts over one device share its queue: work submitted from one
    is visible to the other's later submit without a sync in between.  A
    command whose buffer was freed fails at submit instead of touching it."""
    W = pkg.wgx
    a = W.Context(0)
    b = a.shared()
    try:
        x = a.tensor("float32", [1024]).set_data(np.arange(1024, dtype=np.float32))
        y = a.tensor("float32", [1024])
        z = b.tensor("float32", [1024])
        a.copy(x, y)
        b.copy(y, z)
        a.submit()
        b.submit()
        b.sync()
        assert np.array_equal(z.get_data(), np.arange(1024, dtype=np.float32))
        p = a.storage_buffer(64)
        t = a.tensor("float32", [16], buffer=p)
        b.reset()
        b.copy(t, z)
        a.free(p)
        with pytest.raises(W.WgxError, match="destroyed buffer"):
            b.submit()
    finally:
        b.destroy()
        a.destroy()


def test_short_lists_direct_or_graph(pkg, monkeypatch):
    """A two-command list (the paired float32 headline step) gives the same
    bits issued as direct launches (the default below WGX_GRAPH_MIN) and
    through a captured graph (WGX_GRAPH_MIN=0), on every replay, with the
    input overwritten between replays so each replay must read it again."""
    W, I = pkg.wgx, pkg.inputs
    results = {}
    for gmin in ("3", "0"):
        monkeypatch.setenv("WGX_GRAPH_MIN", gmin)
        ctx = W.Context(0)
        try:
            xa = ctx.from_numpy(I.uniform(61, (1, 16, 20, 20), -1, 1), "float32")
            wa = ctx.from_numpy(I.uniform(62, (32, 16, 3, 3), -0.5, 0.5), "float32")
            xb = ctx.from_numpy(I.uniform(63, (1, 32, 20, 20), -1, 1), "float32")
            wb = ctx.from_numpy(I.uniform(64, (64, 32, 3, 3), -0.5, 0.5), "float32")
            ya, yb = ctx.tensor("float32", [1, 32, 20, 20]), ctx.tensor("float32", [1, 64, 10, 10])
            ctx.convolution(xa, wa, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 1, ya)
            ctx.convolution(xb, wb, None, [2, 2], [1, 1], [1, 1], False, [0, 0], 1, yb)
            outs = []
            for rep in range(3):
                xa.set_data(np.asarray(I.uniform(70 + rep, (1, 16, 20, 20), -1, 1), np.float32))
                ctx.submit()
                ctx.sync()
                outs.append((ya.get_data().copy(), yb.get_data().copy()))
            results[gmin] = outs
        finally:
            ctx.destroy()
    for rep, ((a1, b1), (a2, b2)) in enumerate(zip(results["3"], results["0"])):
        assert np.array_equal(a1.view(np.uint32), a2.view(np.uint32)), f"replay {rep}"
        assert np.array_equal(b1.view(np.uint32), b2.view(np.uint32)), f"replay {rep}"
    # each replay read the input written just before it
    assert not np.array_equal(results["0"][0][0], results["0"][1][0])
