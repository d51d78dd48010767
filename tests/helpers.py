"""Shared helpers for the tests: seeded inputs and the f64 references of the reference's own tests."""
import numpy as np

from oracle import oracle as o

values = o.values  # cuda/tests/common/mod.rs:15-25


def values_fast(count: int, seed: int) -> np.ndarray:
    """Same sequence as `values`, vectorised in blocks for large counts."""
    if count <= 4096:
        return o.values(count, seed)
    a, c = 6364136223846793005, 1442695040888963407
    mask = (1 << 64) - 1
    out = np.empty(count, np.float32)
    # powers of the LCG map: state_{k+j} = A_j * state_k + C_j
    block = 4096
    A = np.empty(block, dtype=object)
    Cc = np.empty(block, dtype=object)
    aj, cj = 1, 0
    for j in range(block):
        aj = (aj * a) & mask
        cj = (cj * a + c) & mask
        A[j], Cc[j] = aj, cj
    A64 = np.array([int(v) for v in A], dtype=np.uint64)
    C64 = np.array([int(v) for v in Cc], dtype=np.uint64)
    state = np.uint64(seed & mask)
    with np.errstate(over="ignore"):
        for s in range(0, count, block):
            n = min(block, count - s)
            st = A64[:n] * state + C64[:n]
            out[s:s + n] = ((st >> np.uint64(40)).astype(np.float32) / np.float32(16777216.0)) * np.float32(2.0) \
                - np.float32(1.0)
            state = st[n - 1]
    return out


def assert_close(actual, expected, tol):
    """cuda/tests/common/mod.rs:27-35: |a - e| <= tol * (1 + |e|)."""
    a, e = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    bad = np.abs(a - e) > tol * (1 + np.abs(e))
    if bad.any():
        i = int(np.argmax(bad))
        raise AssertionError(f"element {i}: gpu {a.flat[i]} vs cpu {e.flat[i]} ({int(bad.sum())} bad)")


def reference_matmul(codes, scales, rows, cols, bits, group, x, tokens):
    """cuda/tests/quant.rs:19-37: dequantized rows dotted with every token in f64."""
    deq = o.dequantize(codes, scales, rows, cols, bits, group).astype(np.float64)
    xs = np.asarray(x, np.float64).reshape(tokens, cols)
    return (xs @ deq.T).astype(np.float32).ravel()


def reference_attention(q, keys, vals, heads, kv_heads, head_dim, start, tokens):
    """cuda/tests/attention_reference/mod.rs:1-49 (the oracle's f64 restatement)."""
    return o.attention(q, keys, vals, heads, kv_heads, head_dim, start, tokens, f64=True)
