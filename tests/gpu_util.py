"""Shared helpers for the GPU parity tests.

Tolerances (written here once, used by every parity test):
  * float32:  |y - y64| <= 1e-5 * sqrt(K) * (|A|.|B|)_ij          (componentwise)
  * float16:  |y - y64| <= 1e-2 * (|A|.|B|)_ij, fp32 accumulation  (componentwise)
  * bfloat16: |y - y64| <= 2e-2 * (|A|.|B|)_ij (8-bit significand output)
where y64 is the oracle's fp64 brute force on the same (already rounded)
inputs and (|A|.|B|)_ij is the oracle's magnitude sum, including |bias|.
"""
import numpy as np


def rel_tol(dtype: str, K: int) -> float:
    if dtype == "float32":
        return 1e-5 * np.sqrt(max(K, 1))
    if dtype == "float16":
        return 1e-2
    return 2e-2


def round_in(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 host data to the storage dtype, returned as float32."""
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
        return r.astype(np.uint32).view(np.float32)
    return x.astype(np.float32)


def assert_parity(y, ref, refabs, dtype, K, what, atol=1e-6):
    y = np.asarray(y, np.float64)
    assert y.shape == ref.shape, f"{what}: shape {y.shape} != {ref.shape}"
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    err = np.abs(y - ref)
    bound = rel_tol(dtype, K) * refabs + atol
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {err.size} outside the {dtype} bound; "
                             f"worst at {i}: got {y[i]!r} expected {ref[i]!r} bound {bound[i]:.3e}")
    return float(np.max(err / np.maximum(refabs, 1e-30)))


def normwise(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))


def sample_rows(M: int, n: int = 96, tile: int = 256) -> np.ndarray:
    """Rows covering every position inside a tile and both matrix edges."""
    rs = np.random.default_rng(M)
    rows = set(range(min(8, M))) | set(range(max(0, M - 8), M))
    rows |= set(int(r) for r in rs.integers(0, M, n))
    rows |= set(range(0, M, max(1, tile // 8 + 1)))
    return np.array(sorted(rows), dtype=np.int32)
