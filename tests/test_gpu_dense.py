"""GPU parity of the dense bf16 half of the boundary (mirrors crates/cuda/tests/ops.rs:15-260): upload_matrix,
matmul on both kernels (the matrix-core one from 16 tokens with columns a multiple of 16), matmul_precise, the
grouped pair/triple (the same bits as separate launches), embed, and the context accessors. The reference product is
f64 over the bf16 weights, tolerance 1e-4 (1 + |e|) as in ops.rs:52."""
import numpy as np
import pytest

import marin_amd as m
from helpers import assert_close, values
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def bf16_bits(v):  # ops.rs:10-13: truncation to bf16
    return o.bf16_bits(v)


def reference(bits, x, rows, cols, tokens):
    w = o.bf16_to_f32(bits).astype(np.float64).reshape(rows, cols)
    return (np.asarray(x, np.float64).reshape(tokens, cols) @ w.T).astype(np.float32).ravel()


def test_buffers_round_trip_and_ranges_are_checked(gpu):  # ops.rs:15-23
    data = np.arange(8, dtype=np.float32)
    b = gpu.upload(data)
    assert np.array_equal(gpu.download(b), data)
    assert np.array_equal(gpu.download_range(b, 2, 3), data[2:5])
    with pytest.raises(m.Shape):
        gpu.download_range(b, 8, 3)
    with pytest.raises(m.Shape):
        gpu.upload_matrix(2, 3, np.zeros(5, np.uint16))


@pytest.mark.parametrize("rows,cols,tokens", [(5, 64, 1), (70, 64, 8), (9, 13, 11), (33, 24, 17), (4, 256, 3),
                                              (9, 16, 16), (70, 48, 65), (130, 256, 129), (64, 2048, 64),
                                              (33, 24, 40), (4096, 4096, 1), (1000, 2048, 4), (512, 4096, 200)])
@pytest.mark.parametrize("precise", [False, True])
def test_matmul_matches_the_cpu_for_aligned_and_odd_shapes_and_token_tiles(gpu, rows, cols, tokens, precise):
    # ops.rs:26-54 (the last three: decode and prompt shapes of a bf16 model)
    weights = bf16_bits(values(rows * cols, 7) if rows * cols <= 1 << 16 else
                        np.random.default_rng(7).uniform(-1, 1, rows * cols).astype(np.float32))
    x = values(tokens * cols, 9) if tokens * cols <= 1 << 16 else \
        np.random.default_rng(9).uniform(-1, 1, tokens * cols).astype(np.float32)
    w = gpu.upload_matrix(rows, cols, weights)
    out = gpu.zeros(tokens * rows)
    (gpu.matmul_precise if precise else gpu.matmul)(w, gpu.upload(x), tokens, out)
    assert_close(gpu.download(out), reference(weights, x, rows, cols, tokens), 1e-4)


def grouped_case(gpu, rows, cols, tokens):  # ops.rs:57-96
    x = gpu.upload(values(tokens * cols, 51))
    ws = [gpu.upload_matrix(r, cols, bf16_bits(values(r * cols, 60 + i))) for i, r in enumerate(rows)]
    separate = [gpu.zeros(tokens * r) for r in rows]
    for w, out in zip(ws, separate):
        gpu.matmul(w, x, tokens, out)
    grouped = [gpu.zeros(tokens * r) for r in rows]
    (gpu.matmul_pair if len(rows) == 2 else gpu.matmul_triple)(ws, x, tokens, grouped)
    for a, b in zip(grouped, separate):
        assert np.array_equal(gpu.download(a).view(np.uint32), gpu.download(b).view(np.uint32)), (rows, cols, tokens)


def test_grouped_matmuls_give_the_same_bits_as_separate_ones(gpu):  # ops.rs:97-110
    for tokens in (1, 3, 8, 9, 15, 16, 40):
        for cols in (64, 13, 2048):
            grouped_case(gpu, [5, 7], cols, tokens)
            grouped_case(gpu, [6, 1, 9], cols, tokens)
    grouped_case(gpu, [128, 64, 64], 128, 1)
    grouped_case(gpu, [96, 96], 64, 2)


def test_grouped_matmuls_reject_mismatched_shapes_instead_of_launching(gpu):  # ops.rs:112-143
    def w(r, c):
        return gpu.upload_matrix(r, c, np.zeros(r * c, np.uint16))
    x = gpu.zeros(8)
    a, b = gpu.zeros(2), gpu.zeros(3)
    with pytest.raises(m.Shape):
        gpu.matmul_pair((w(2, 8), w(3, 4)), x, 1, (a, b))
    with pytest.raises(m.Shape):
        gpu.matmul_pair((w(2, 8), w(4, 8)), x, 1, (a, b))
    with pytest.raises(m.Shape):
        gpu.matmul_pair((w(2, 8), w(3, 8)), gpu.zeros(7), 1, (a, b))
    gpu.matmul_pair((w(2, 8), w(3, 8)), x, 1, (a, b))


def test_matmul_rejects_wrongly_sized_buffers_instead_of_launching(gpu):  # ops.rs:145-154
    w = gpu.upload_matrix(2, 8, np.zeros(16, np.uint16))
    x = gpu.upload(np.zeros(8, np.float32))
    with pytest.raises(m.Shape):
        gpu.matmul(w, x, 1, gpu.zeros(1))
    with pytest.raises(m.Shape):
        gpu.matmul(w, x, 2, gpu.zeros(2))


def test_embed_matches_the_table_and_refuses_what_it_cannot_hold(gpu):  # ops.rs:232-254
    table_values = values(10 * 16, 13)
    bits = bf16_bits(table_values)
    table = gpu.upload_matrix(10, 16, bits)
    rows = o.bf16_to_f32(bits).reshape(10, 16)
    out = gpu.zeros(3 * 16)
    ids = gpu.tokens(4)
    gpu.embed(table, [4, 0, 9], ids, out)
    expected = np.concatenate([rows[4], rows[0], rows[9]])
    assert np.array_equal(gpu.download(out).view(np.uint32), expected.view(np.uint32))
    one = gpu.zeros(16)
    gpu.embed(table, [9], ids, one)
    assert np.array_equal(gpu.download(one), expected[32:])
    with pytest.raises(m.Shape):
        gpu.embed(table, [10], ids, one)
    with pytest.raises(m.Shape):
        gpu.embed(table, [0] * 5, ids, gpu.zeros(5 * 16))


def test_reports_the_device_and_binds_to_a_thread(gpu):  # ops.rs:256-265, gpu.rs:238-242
    import threading
    info = gpu.info()
    assert info["name"] and info["total_bytes"] >= info["free_bytes"]
    errors = []

    def work():
        try:
            gpu.bind_to_thread()
            b = gpu.upload([1.0, 2.0])
            assert gpu.download(b).tolist() == [1.0, 2.0]
        except Exception as e:  # noqa: BLE001
            errors.append(e)
    t = threading.Thread(target=work)
    t.start()
    t.join()
    assert not errors, errors


@pytest.mark.parametrize("fmt", [m.KvFormat.F32, m.KvFormat.F16])
def test_a_cache_reports_its_format_emptiness_and_auxiliary_bytes(gpu, fmt):  # kv.rs:81-150
    kv = m.DeviceKv(gpu, 2, (4, 2, 16), 300, fmt)
    assert kv.kv_format() == fmt and kv.is_empty()
    aux = kv.auxiliary_bytes()
    # the page table alone is 8 bytes per page of the capacity; the split scratch comes on top
    assert aux >= m.pages_for(300) * 8
    kv.write(gpu, 0, gpu.zeros(5 * 32), gpu.zeros(5 * 32))
    kv.advance(5)
    assert not kv.is_empty() and kv.auxiliary_bytes() == aux
    startup = m.DeviceKv.startup_bytes(2, (4, 2, 16), 300, fmt)
    assert startup >= kv.slab_bytes() + m.pages_for(300) * 8
