"""wgx_mm_noalloc: the mm / addmm launched at once with its workspace in the
library's fixed per-device scratch array (no device allocation).

Each case runs twice in a row on one device, the second time with a smaller
input, and each result must equal, bit for bit, what wgx_record_mm computes
on the same inputs (the same kernels read the same values; only where the
workspace lives differs).  The cases use both kinds of workspace: the [N, K]
staging copy of a 16-bit [K, N] B (large-tile kernel) and split-K partial
sums.  A GEMM whose workspace exceeds the array is refused before launch.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pair(ctx, I, dtype, M, K, N, seed, bias=True):
    A = I.normal(seed, (M, K))
    B = I.normal(seed + 1, (K, N), 0.0, 0.05)
    b = I.uniform(seed + 2, (N,), -0.1, 0.1) if bias else None
    ta, tb = ctx.from_numpy(A, dtype), ctx.from_numpy(B, dtype)
    tbias = ctx.from_numpy(b, dtype) if bias else None
    rec, nal = ctx.tensor(dtype, [M, N]), ctx.tensor(dtype, [M, N])
    ctx.reset()
    ctx.mm(ta, tb, rec, bias=tbias)
    recorded_kernel = ctx.last_kernel
    ctx.submit()
    ctx.sync()
    ctx.mm_noalloc(ta, tb, nal, bias=tbias)
    noalloc_kernel = ctx.last_kernel
    ctx.sync()
    return rec.get_data(), nal.get_data(), recorded_kernel, noalloc_kernel


# (dtype, first (M, K, N), second smaller (M, K, N), kernel-name marker of the workspace)
CASES = [
    ("float16", (4096, 768, 3072), (4096, 512, 3072), "kn2nk_big"),  # [N, K] staging copy of B
    ("bfloat16", (128, 4096, 128), (64, 2048, 64), "_k"),            # split-K partial sums
]


@pytest.mark.parametrize("dtype,first,second,marker", CASES, ids=["staging", "splitk"])
def test_mm_noalloc_matches_recorded_twice(pkg, dtype, first, second, marker):
    W, I = pkg.wgx, pkg.inputs
    ctx = W.Context(0)
    try:
        for seed, (M, K, N) in ((80, first), (90, second)):
            print(f"[mm_noalloc] {dtype} M={M} K={K} N={N}", flush=True)
            rec, nal, krec, knal = _pair(ctx, I, dtype, M, K, N, seed)
            assert krec == knal, (krec, knal)
            if (M, K, N) == first:
                assert marker in knal, knal
            assert np.array_equal(rec.view(np.uint16), nal.view(np.uint16)), f"{knal}: differs from the recorded GEMM"
    finally:
        ctx.destroy()


def test_mm_noalloc_refuses_oversized_workspace(pkg):
    W, I = pkg.wgx, pkg.inputs
    ctx = W.Context(0)
    try:
        # a 2048 x 3072 [K, N] float16 B on the large-tile kernel needs a
        # 12 MiB [N, K] staging copy
        ta = ctx.tensor("float16", [4096, 2048])
        tb = ctx.tensor("float16", [2048, 3072])
        to = ctx.tensor("float16", [4096, 3072])
        with pytest.raises(W.WgxError, match="needs 12582912 bytes of workspace; the fixed scratch holds 8388608"):
            ctx.mm_noalloc(ta, tb, to)
        ctx.reset()
        ctx.mm(ta, tb, to)
        assert "kn2nk_big" in ctx.last_kernel  # the recorded form stages it in its own workspace
        # float32 and small 16-bit GEMMs need none and run
        A = I.uniform(95, (64, 96), -1, 1)
        B = I.uniform(96, (96, 80), -1, 1)
        x, y = ctx.from_numpy(A, "float32"), ctx.from_numpy(B, "float32")
        o1, o2 = ctx.tensor("float32", [64, 80]), ctx.tensor("float32", [64, 80])
        ctx.reset()
        ctx.mm(x, y, o1)
        ctx.submit()
        ctx.mm_noalloc(x, y, o2)
        ctx.sync()
        assert np.array_equal(o1.get_data(), o2.get_data())
    finally:
        ctx.destroy()
