"""Pins the CPU oracle before anything is compared against it.

Each check is chosen so a plausible mistake in the oracle (a dropped bias, a
transposed operand, an off-by-one pad or stride, a wrong rounding rule) fails
at least one of them:
  * the reference's own known-answer tests (tests/golden/reference_kats.json),
  * torch float64 on the CPU as an independent library,
  * numpy float16 scalar arithmetic as an independent f16 rounding model,
  * closed forms (A.I = A, identity 1x1, one-hot depthwise = shift),
  * planted mistakes: a deliberately wrong oracle call must fail the KATs.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F


def _arr(t, dtype=np.float32):
    return np.asarray(t["data"], dtype=dtype).reshape(t["shape"])


def _as_dtype(x, dt):
    return x.astype(np.float16).astype(np.float32) if dt == "float16" else x.astype(np.float32)


# ------------------------------------------------------------ number formats
def test_f16_conversion_matches_numpy_all_halves(orc):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = orc.f16_bits_to_f32(h)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy(orc):
    rs = np.random.default_rng(1)
    bits = rs.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # ties and the overflow / subnormal boundaries explicitly
    edge = np.array([65504, 65519.99, 65520, 65536, 6.1035156e-05, 6.097555e-05, 5.9604645e-08,
                     2.9802322e-08, 2.9802326e-08, 1.0 + 2**-11, 1.0 + 3 * 2**-11, -0.0, np.inf,
                     -np.inf], dtype=np.float32)
    x = np.concatenate([x, edge, -edge])
    with np.errstate(all="ignore"):
        ref = x.astype(np.float16)
    got = orc.f32_to_f16_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan].view(np.uint16))
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_bf16_conversion_matches_torch(orc):
    rs = np.random.default_rng(2)
    x = rs.standard_normal(200_000).astype(np.float32) * 1e3
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16_bits(x), ref)
    back = orc.bf16_bits_to_f32(ref)
    assert np.array_equal(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


# ------------------------------------------------------------ reference KATs
def _run_kat_f64(orc, c):
    if c["op"] == "aten.mm.default":
        a, b = _as_dtype(_arr(c["a"]), c["dtype"]), _as_dtype(_arr(c["b"]), c["dtype"])
        return orc.gemm_f64(a, b)[0], a.astype(np.float64) @ b.astype(np.float64)
    if c["op"] == "aten.bmm.default":
        a, b = _as_dtype(_arr(c["a"]), c["dtype"]), _as_dtype(_arr(c["b"]), c["dtype"])
        return orc.gemm_f64(a, b)[0], np.matmul(a.astype(np.float64), b.astype(np.float64))
    if c["op"] == "aten.convolution.default":
        x, w = _as_dtype(_arr(c["input"]), c["dtype"]), _as_dtype(_arr(c["weight"]), c["dtype"])
        b = _as_dtype(_arr(c["bias"]), c["dtype"]) if c["bias"] else None
        kw = dict(stride=c["stride"], padding=c["padding"], dilation=c["dilation"], groups=c["groups"])
        if c["transposed"]:
            y = orc.conv_transpose2d_f64(x, w, b, output_padding=c["output_padding"], **kw)[0]
        else:
            y = orc.conv2d_f64(x, w, b, **kw)[0]
        assert list(y.shape) == c["out_shape"]
        return y, None
    raise AssertionError(c["op"])


def test_reference_kats_fp64(orc, kats):
    n = 0
    for c in kats:
        if c["op"] == "program":
            continue
        got, closed = _run_kat_f64(orc, c)
        if c["expected"] is not None:
            exp = np.asarray(c["expected"], np.float64)
            assert np.max(np.abs(got.ravel() - exp)) <= c["tol"], c["source"]
        elif "identity" in c.get("check", ""):
            assert np.max(np.abs(got - _arr(c["b"]))) <= c["tol"], c["source"]
        elif closed is not None:
            assert np.array_equal(got, closed), c["source"]  # integer data: exact
        else:  # "element 0" checks of the 1x1 conv tests
            x, w = _arr(c["input"]), _arr(c["weight"])
            e0 = sum(float(x.ravel()[ic * 64]) * float(w.ravel()[ic]) for ic in range(x.shape[1]))
            assert abs(got.ravel()[0] - e0) <= c["tol"], c["source"]
        n += 1
    assert n == 21


def test_reference_kats_emu(orc, kats):
    """The WGSL restatement also reproduces every KAT (f16 cases in f16)."""
    for c in kats:
        if c["op"] == "program" or c["expected"] is None:
            continue
        dt = 1 if c["dtype"] == "float16" else 0
        if c["op"] in ("aten.mm.default", "aten.bmm.default"):
            a, b = _as_dtype(_arr(c["a"]), c["dtype"]), _as_dtype(_arr(c["b"]), c["dtype"])
            got = orc.emu_gemm(dt, a, b)
        else:
            x, w = _as_dtype(_arr(c["input"]), c["dtype"]), _as_dtype(_arr(c["weight"]), c["dtype"])
            b = _as_dtype(_arr(c["bias"]), c["dtype"]) if c["bias"] else None
            got = orc.emu_conv2d(dt, x, w, b, c["stride"], c["padding"], c["dilation"], c["groups"],
                                 c["transposed"], c["output_padding"])
        exp = np.asarray(c["expected"], np.float64)
        assert np.max(np.abs(got.ravel() - exp)) <= max(c["tol"], 1e-4), c["source"]


def test_program_kat(orc, kats):
    c = [k for k in kats if k["op"] == "program"][0]
    a, b, cc = (np.asarray(c[k], np.float32).reshape(2, 2) for k in "abc")
    t = a + np.float32(c["alpha"]) * b
    out = orc.gemm_f64(t, cc)[0]
    assert np.array_equal(out.ravel(), np.asarray(c["expected"], np.float64))


# ------------------------------------------------------------ planted mistakes
def test_planted_mistakes_fail_the_kats(orc, kats):
    strided = [c for c in kats if c["source"].endswith(":132-176")][0]
    x, w, b = _arr(strided["input"]), _arr(strided["weight"]), _arr(strided["bias"])
    exp = np.asarray(strided["expected"])
    good = orc.conv2d_f64(x, w, b, stride=(2, 2), padding=(1, 1))[0].ravel()
    assert np.max(np.abs(good - exp)) < 1e-3
    wrong = [
        orc.conv2d_f64(x, w, None, stride=(2, 2), padding=(1, 1))[0],          # dropped bias
        orc.conv2d_f64(x, w, b, stride=(2, 2), padding=(0, 0))[0],             # pad off by one
        orc.conv2d_f64(x, w[:, :, ::-1, ::-1].copy(), b, stride=(2, 2), padding=(1, 1))[0],  # flipped kernel
        orc.conv2d_f64(x.transpose(0, 1, 3, 2).copy(), w, b, stride=(2, 2), padding=(1, 1))[0],  # H/W swapped
    ]
    for y in wrong:
        assert y.size != exp.size or np.max(np.abs(y.ravel() - exp)) > 1.0
    mm = [c for c in kats if c["source"] == "tests/shaders/bmm.test.ts:6-23"][0]
    a, bb = _arr(mm["a"])[0], _arr(mm["b"])[0]
    assert not np.allclose(orc.gemm_f64(bb.T.copy(), a.T.copy())[0].ravel(), mm["expected"])


# ------------------------------------------------------------ torch float64 cross-checks
CONV_CASES = [
    # x shape, w shape, stride, pad, dil, groups
    ((1, 3, 11, 9), (5, 3, 3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((2, 4, 10, 10), (6, 4, 3, 3), (2, 2), (1, 1), (1, 1), 1),
    ((1, 6, 9, 12), (6, 2, 3, 2), (1, 2), (0, 1), (2, 1), 3),
    ((2, 8, 13, 7), (8, 1, 5, 5), (2, 2), (2, 2), (1, 1), 8),
    ((1, 5, 6, 6), (7, 5, 1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 3, 8, 8), (4, 3, 7, 7), (1, 1), (3, 3), (1, 1), 1),
]


@pytest.mark.parametrize("xs,ws,s,p,d,g", CONV_CASES)
def test_conv2d_f64_matches_torch(orc, xs, ws, s, p, d, g):
    rs = np.random.default_rng(hash((xs, ws)) & 0xFFFF)
    x = rs.uniform(-1, 1, xs).astype(np.float32)
    w = rs.uniform(-1, 1, ws).astype(np.float32)
    b = rs.uniform(-1, 1, ws[0]).astype(np.float32)
    y, ya = orc.conv2d_f64(x, w, b, s, p, d, g)
    ref = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                   torch.from_numpy(b).double(), s, p, d, g).numpy()
    assert y.shape == ref.shape
    assert np.max(np.abs(y - ref)) < 1e-12
    refa = F.conv2d(torch.from_numpy(np.abs(x)).double(), torch.from_numpy(np.abs(w)).double(),
                    torch.from_numpy(np.abs(b)).double(), s, p, d, g).numpy()
    assert np.max(np.abs(ya - refa)) < 1e-12


@pytest.mark.parametrize("xs,ws,s,p,d,g,op", [
    ((1, 2, 3, 3), (2, 3, 3, 3), (2, 2), (1, 1), (1, 1), 1, (1, 1)),
    ((2, 4, 5, 4), (4, 2, 2, 3), (2, 1), (0, 1), (1, 2), 2, (1, 0)),
    ((1, 3, 4, 4), (3, 1, 4, 4), (2, 2), (1, 1), (1, 1), 1, (0, 0)),
])
def test_conv_transpose2d_f64_matches_torch(orc, xs, ws, s, p, d, g, op):
    rs = np.random.default_rng(7)
    x = rs.uniform(-1, 1, xs).astype(np.float32)
    w = rs.uniform(-1, 1, ws).astype(np.float32)
    b = rs.uniform(-1, 1, ws[1] * g).astype(np.float32)
    y, _ = orc.conv_transpose2d_f64(x, w, b, s, p, d, g, op)
    ref = F.conv_transpose2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                             torch.from_numpy(b).double(), s, p, op, g, d).numpy()
    assert y.shape == ref.shape and np.max(np.abs(y - ref)) < 1e-12
    ye = orc.emu_conv2d(0, x, w, b, s, p, d, g, transposed=True, output_padding=op)
    assert np.max(np.abs(ye - ref)) < 1e-5


def test_gemm_f64_forms_match_numpy(orc):
    rs = np.random.default_rng(3)
    A = rs.uniform(-1, 1, (37, 53)).astype(np.float32)
    B = rs.uniform(-1, 1, (53, 29)).astype(np.float32)
    bias = rs.uniform(-1, 1, 29).astype(np.float32)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    C, Ca = orc.gemm_f64(A, B)
    assert np.max(np.abs(C - ref)) < 1e-12
    assert np.max(np.abs(Ca - np.abs(A).astype(np.float64) @ np.abs(B))) < 1e-12
    Ct, _ = orc.gemm_f64(A, B.T.copy(), b_trans=True)
    assert np.max(np.abs(Ct - ref)) < 1e-12
    Cb, _ = orc.gemm_f64(A, B, bias)
    assert np.max(np.abs(Cb - (ref + bias))) < 1e-12
    rows = [0, 5, 36]
    Cr, _ = orc.gemm_f64(A, B, bias, rows=rows)
    assert np.max(np.abs(Cr - (ref + bias)[rows])) < 1e-12
    A3 = rs.uniform(-1, 1, (3, 8, 5)).astype(np.float32)
    B3 = rs.uniform(-1, 1, (3, 5, 6)).astype(np.float32)
    C3, _ = orc.gemm_f64(A3, B3)
    assert np.max(np.abs(C3 - np.matmul(A3.astype(np.float64), B3))) < 1e-12


def test_gemm_identity_closed_form(orc):
    rs = np.random.default_rng(4)
    A = rs.uniform(-1, 1, (16, 16)).astype(np.float32)
    I = np.eye(16, dtype=np.float32)
    assert np.array_equal(orc.gemm_f64(A, I)[0], A.astype(np.float64))
    assert np.array_equal(orc.emu_gemm(0, A, I), A)
    assert np.array_equal(orc.emu_gemm(1, A.astype(np.float16).astype(np.float32), I),
                          A.astype(np.float16).astype(np.float32))


def test_depthwise_one_hot_is_shift(orc):
    rs = np.random.default_rng(5)
    x = rs.uniform(-1, 1, (1, 4, 9, 9)).astype(np.float32)
    w = np.zeros((4, 1, 3, 3), np.float32)
    w[:, 0, 0, 2] = 1.0  # tap (kh=0, kw=2) -> y[h,w] = x[h-1, w+1]
    y, _ = orc.conv2d_f64(x, w, None, padding=(1, 1), groups=4)
    shifted = np.zeros_like(x, dtype=np.float64)
    shifted[:, :, 1:, :-1] = x[:, :, :-1, 1:]
    assert np.array_equal(y, shifted)


# ------------------------------------------------------------ f16 emulation vs numpy.float16
def _np16_seq_dot(a_row, b_col, init=np.float16(0)):
    acc = np.float16(init)
    for av, bv in zip(a_row, b_col):
        acc = np.float16(acc + np.float16(np.float16(av) * np.float16(bv)))
    return acc


def test_emu_gemm_f16_matches_numpy_float16_loop(orc):
    rs = np.random.default_rng(6)
    A = rs.standard_normal((5, 96)).astype(np.float16)
    B = (rs.standard_normal((96, 7)) * 0.02).astype(np.float16)
    got = orc.emu_gemm(1, A.astype(np.float32), B.astype(np.float32))
    for i in range(5):
        for j in range(7):
            assert got[i, j] == np.float32(_np16_seq_dot(A[i], B[:, j]))
    gt = orc.emu_gemm(1, A.astype(np.float32), B.T.astype(np.float32).copy(), b_trans=True)
    assert np.array_equal(gt, got)
    bias = rs.uniform(-0.1, 0.1, 7).astype(np.float16)
    am = orc.emu_addmm(1, A.astype(np.float32), B.astype(np.float32), bias.astype(np.float32))
    assert np.array_equal(am, (got.astype(np.float16) + bias).astype(np.float32))


def test_emu_depthwise_f16_matches_numpy_float16_loop(orc):
    rs = np.random.default_rng(8)
    x = rs.standard_normal((1, 3, 7, 6)).astype(np.float16)
    w = rs.uniform(-0.5, 0.5, (3, 1, 5, 5)).astype(np.float16)
    bias = rs.uniform(-0.1, 0.1, 3).astype(np.float16)
    got = orc.emu_conv2d(1, x.astype(np.float32), w.astype(np.float32), bias.astype(np.float32),
                         stride=(2, 2), padding=(2, 2), groups=3)
    OH, OW = got.shape[2:]
    for c in range(3):
        for oh in range(OH):
            for ow in range(OW):
                acc = bias[c]
                for kh in range(5):
                    for kw in range(5):
                        ih, iw = oh * 2 - 2 + kh, ow * 2 - 2 + kw
                        if 0 <= ih < 7 and 0 <= iw < 6:
                            acc = np.float16(acc + np.float16(x[0, c, ih, iw] * w[c, 0, kh, kw]))
                assert got[0, c, oh, ow] == np.float32(acc)


def test_emu_dense_conv_f16_bias_last(orc):
    rs = np.random.default_rng(9)
    x = rs.standard_normal((1, 2, 5, 5)).astype(np.float16)
    w = rs.uniform(-0.5, 0.5, (3, 2, 3, 3)).astype(np.float16)
    bias = rs.uniform(-1, 1, 3).astype(np.float16)
    got = orc.emu_conv2d(1, x.astype(np.float32), w.astype(np.float32), bias.astype(np.float32),
                         padding=(1, 1))
    for oc in range(3):
        for oh in range(5):
            for ow in range(5):
                acc = np.float16(0)
                for ic in range(2):
                    for kh in range(3):
                        for kw in range(3):
                            ih, iw = oh - 1 + kh, ow - 1 + kw
                            if 0 <= ih < 5 and 0 <= iw < 5:
                                acc = np.float16(acc + np.float16(x[0, ic, ih, iw] * w[oc, ic, kh, kw]))
                assert got[0, oc, oh, ow] == np.float32(np.float16(acc + bias[oc]))


def test_emu_f32_gemm_within_fp64_bound(orc):
    rs = np.random.default_rng(10)
    A = rs.uniform(-1, 1, (64, 512)).astype(np.float32)
    B = rs.uniform(-1, 1, (512, 48)).astype(np.float32)
    C, Ca = orc.gemm_f64(A, B)
    E = orc.emu_gemm(0, A, B)
    assert np.all(np.abs(E - C) <= 512 * 2**-24 * Ca)


# ------------------------------------------------------------ oracle/ops.py pins
def test_max_pool_kats_and_torch(orc):
    """max_pool2d_with_indices: the reference KATs (tests/shaders/max-pool-2d.test.ts:6-44),
    torch's values and indices on tie-free inputs, and the first-of-equal rule
    on a constant plane (closed form: the first in-image cell of each window)."""
    from oracle import ops

    x = np.arange(1, 17, dtype=np.float64).reshape(1, 1, 4, 4)
    v, i = ops.max_pool2d_with_indices(x, (2, 2), (2, 2), (0, 0), (1, 1))
    assert v.ravel().tolist() == [6, 8, 14, 16] and i.ravel().tolist() == [5, 7, 13, 15]
    v, i = ops.max_pool2d_with_indices(np.array([1, 2, 3, 4.0]).reshape(1, 1, 2, 2), (3, 3), (1, 1), (1, 1), (1, 1))
    assert v.ravel().tolist() == [4, 4, 4, 4] and i.ravel().tolist() == [3, 3, 3, 3]
    rs = np.random.default_rng(5)
    for shape, k, s, p, d in [((2, 3, 17, 23), (3, 3), (2, 2), (1, 1), (1, 1)),
                              ((1, 4, 16, 15), (2, 3), (2, 1), (0, 1), (2, 1)),
                              ((1, 128, 20, 20), (5, 5), (1, 1), (2, 2), (1, 1)),
                              ((1, 2, 9, 9), (4, 4), (3, 3), (1, 2), (1, 1))]:
        x = rs.permutation(int(np.prod(shape))).astype(np.float64).reshape(shape)  # distinct values
        for ceil in (False, True):
            v, i = ops.max_pool2d_with_indices(x, k, s, p, d, ceil)
            tv, ti = F.max_pool2d(torch.from_numpy(x), k, s, p, d, ceil_mode=ceil, return_indices=True)
            if tuple(tv.shape) != v.shape:  # torch drops a last window that starts in the padding
                continue
            assert np.array_equal(v, tv.numpy()) and np.array_equal(i, ti.numpy())
    c = np.full((1, 1, 5, 7), 3.0)
    v, i = ops.max_pool2d_with_indices(c, (3, 3), (2, 2), (1, 1), (1, 1))
    for oh in range(v.shape[2]):
        for ow in range(v.shape[3]):
            assert i[0, 0, oh, ow] == max(0, oh * 2 - 1) * 7 + max(0, ow * 2 - 1)
    # -inf and NaN never win; a window with nothing greater than the floor keeps it
    y = np.array([[[[-np.inf, np.nan], [np.nan, -np.inf]]]])
    v, i = ops.max_pool2d_with_indices(y, (2, 2), (1, 1), (0, 0), (1, 1), dtype="float16")
    assert v.ravel().tolist() == [-65504.0] and i.ravel().tolist() == [0]
    assert ops.pool_out_size(3, 2, 2, 0, 1, True) == 2 and ops.pool_out_size(3, 2, 2, 0, 1, False) == 1


def test_softmax_and_permute_pins(orc):
    """softmax_f64 against torch (float64) and the reference KATs
    (tests/shaders/softmax.test.ts:6-80); permute against the reference KATs
    (tests/shaders/permute.test.ts:6-69)."""
    from oracle import ops

    rs = np.random.default_rng(6)
    for shape, dim in [((1, 2, 3), -1), ((2, 2), 0), ((3, 7, 5), 1), ((2, 400, 400), 2)]:
        x = rs.standard_normal(shape) * 4
        assert np.allclose(ops.softmax_f64(x, dim), torch.softmax(torch.from_numpy(x), dim).numpy(), rtol=1e-13, atol=0)
        assert np.allclose(ops.softmax_f64(x, dim).sum(axis=dim), 1.0)
    e = np.exp([1.0, 2, 3])
    assert np.allclose(ops.softmax_f64(np.array([[1.0, 2, 3]]), -1), e / e.sum(), rtol=1e-15)
    assert np.allclose(ops.softmax_f64(np.array([[1.0, 2], [3, 4]]), 0).ravel(),
                       [np.exp(1) / (np.exp(1) + np.exp(3)), np.exp(2) / (np.exp(2) + np.exp(4)),
                        np.exp(3) / (np.exp(1) + np.exp(3)), np.exp(4) / (np.exp(2) + np.exp(4))])
    assert ops.permute(np.arange(1, 7).reshape(2, 3), [1, 0]).ravel().tolist() == [1, 4, 2, 5, 3, 6]
    assert ops.permute(np.arange(1, 13).reshape(1, 2, 2, 3), [0, 1, 3, 2]).ravel().tolist() == \
        [1, 4, 2, 5, 3, 6, 7, 10, 8, 11, 9, 12]
    m = np.array([[r * 100 + c for c in range(48)] for r in range(64)])
    assert np.array_equal(ops.permute(m, [1, 0]), m.T)
    with pytest.raises(ValueError):
        ops.permute(m, [0, 0])
