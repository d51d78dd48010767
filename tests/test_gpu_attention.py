"""GPU parity of the paged KV cache and decode attention (mirrors crates/cuda/tests/attention.rs, paging.rs,
mirror/mod.rs, kv_formats.rs) against the f64 attention of cuda/tests/attention_reference/mod.rs."""
import numpy as np
import pytest

import marin_amd as m
from oracle import oracle as o
from helpers import assert_close, reference_attention, values

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("head_dim,history,tokens", [
    (16, 0, 1), (16, 97, 3), (16, 5, 9), (64, 40, 4), (128, 70, 2), (128, 0, 40), (128, 300, 12), (64, 127, 16),
    (16, 129, 9), (16, 255, 11), (30, 130, 9), (18, 260, 10), (10, 130, 9), (13, 70, 9)])
def test_attention_matches_a_reference_across_chunks_and_context_lengths(gpu, head_dim, history, tokens):
    heads, kvh = 4, 2
    stride = kvh * head_dim
    total = history + tokens
    keys = values(total * stride, 21)
    vals = values(total * stride, 22)
    q = values(tokens * heads * head_dim, 23)
    kv = m.DeviceKv(gpu, 2, (heads, kvh, head_dim), total + 3, m.KvFormat.F32)
    if history:
        kv.write(gpu, 1, gpu.upload(keys[:history * stride]), gpu.upload(vals[:history * stride]))
        kv.advance(history)
    kv.write(gpu, 1, gpu.upload(keys[history * stride:]), gpu.upload(vals[history * stride:]))
    out = gpu.zeros(q.size)
    gpu.attention(gpu.upload(q), kv, 1, heads, tokens, out)
    assert_close(gpu.download(out), reference_attention(q, keys, vals, heads, kvh, head_dim, history, tokens), 1e-4)


def f16_round(x):
    """cuda/tests/kv_round/mod.rs:3-18"""
    return np.clip(np.asarray(x, np.float32), -65504, 65504).astype(np.float16).astype(np.float32)


def bf16_round(x):
    return o.bf16_to_f32(o.f32_to_bf16_rne(x))


class Mirror:
    """cuda/tests/mirror/mod.rs: a DeviceKv plus a host copy of what it must hold (after the format's rounding)."""
    LAYERS = 2
    SMALL = (4, 2, 16)

    def __init__(self, gpu, dims, capacity, fmt=m.KvFormat.F32):
        self.kv = m.DeviceKv(gpu, self.LAYERS, dims, capacity, fmt)
        self.dims, self.fmt = dims, fmt
        self.keys = [np.zeros(0, np.float32) for _ in range(self.LAYERS)]
        self.vals = [np.zeros(0, np.float32) for _ in range(self.LAYERS)]
        self.seed = 1

    def stride(self):
        return self.dims[1] * self.dims[2]

    def rounded(self, x):
        return {m.KvFormat.F32: lambda v: v, m.KvFormat.F16: f16_round, m.KvFormat.BF16: bf16_round}[self.fmt](x)

    def append(self, gpu, tokens):
        n = tokens * self.stride()
        for layer in range(self.LAYERS):
            self.seed += 1
            k = values(n, 1000 + self.seed) * np.float32(3.0)
            self.seed += 1
            v = values(n, 2000 + self.seed) * np.float32(3.0)
            self.kv.write(gpu, layer, gpu.upload(k), gpu.upload(v))
            self.keys[layer] = np.concatenate([self.keys[layer], self.rounded(k)])
            self.vals[layer] = np.concatenate([self.vals[layer], self.rounded(v)])
        self.kv.advance(tokens)

    def truncate(self, length):
        self.kv.truncate(length)
        for layer in range(self.LAYERS):
            self.keys[layer] = self.keys[layer][:length * self.stride()]
            self.vals[layer] = self.vals[layer][:length * self.stride()]

    def check(self, gpu, tokens):
        """Attends `tokens` new tokens at the end (written, then rolled back), in every layer."""
        heads, kvh, hd = self.dims
        start = self.kv.len()
        if start + tokens > self.kv.capacity():
            return
        n = tokens * self.stride()
        for layer in range(self.LAYERS):
            k = values(n, 31 + layer)
            v = values(n, 41 + layer)
            q = values(tokens * heads * hd, 51 + layer)
            self.kv.write(gpu, layer, gpu.upload(k), gpu.upload(v))
            out = gpu.zeros(q.size)
            gpu.attention(gpu.upload(q), self.kv, layer, heads, tokens, out)
            keys = np.concatenate([self.keys[layer], self.rounded(k)])
            vals = np.concatenate([self.vals[layer], self.rounded(v)])
            assert_close(gpu.download(out), reference_attention(q, keys, vals, heads, kvh, hd, start, tokens), 1e-4)
        self.kv.truncate(start)

    def check_every_kernel(self, gpu):
        for tokens in (1, 3, 8, 12):
            self.check(gpu, tokens)


@pytest.mark.parametrize("total", [0, 1, 2, 31, 32, 33, 62, 63, 64, 65, 66, 126, 127, 128, 129, 130, 191, 192, 193,
                                   320, 321])
def test_attention_reads_the_right_page_and_row_at_every_boundary(gpu, total):  # paging.rs:12-31
    mir = Mirror(gpu, Mirror.SMALL, 400)
    if total:
        mir.append(gpu, total)
    assert mir.kv.pages_in_use() == m.pages_for(total)
    mir.check_every_kernel(gpu)
    assert mir.kv.pages_in_use() == m.pages_for(total)


def test_growing_one_token_at_a_time_crosses_pages(gpu):  # paging.rs:33-47
    mir = Mirror(gpu, Mirror.SMALL, 260)
    for length in range(1, 201):
        mir.append(gpu, 1)
        assert mir.kv.pages_in_use() == m.pages_for(length)
        if length in (1, 63, 64, 65, 127, 128, 129, 191, 192, 193, 200):
            mir.check(gpu, 1)
            mir.check(gpu, 4)


def test_a_realistic_head_layout_reads_pages_correctly(gpu):  # paging.rs:49-58
    for total in (63, 64, 65, 129):
        mir = Mirror(gpu, (16, 8, 128), 300)
        mir.append(gpu, total)
        mir.check_every_kernel(gpu)


def test_a_cleared_and_refilled_cache_reads_through_a_reversed_page_table(gpu):  # paging.rs:60-83
    mir = Mirror(gpu, Mirror.SMALL, 600)
    tokens = 5 * m.PAGE_TOKENS + 17
    mir.append(gpu, tokens)
    assert mir.kv.page_ids() == [0, 1, 2, 3, 4, 5]
    mir.truncate(0)
    assert mir.kv.pages_in_use() == 0
    mir.append(gpu, tokens)
    assert mir.kv.page_ids() == [5, 4, 3, 2, 1, 0]
    mir.check_every_kernel(gpu)
    assert mir.kv.pages_held() == 6


def test_rolling_back_into_a_page_and_regrowing_mixes_the_page_order(gpu):  # paging.rs:101-113
    mir = Mirror(gpu, Mirror.SMALL, 600)
    mir.append(gpu, 400)
    assert mir.kv.page_ids() == [0, 1, 2, 3, 4, 5, 6]
    mir.truncate(70)
    assert mir.kv.page_ids() == [0, 1]
    mir.append(gpu, 330)
    assert mir.kv.page_ids() == [0, 1, 6, 5, 4, 3, 2]
    mir.check_every_kernel(gpu)
    assert mir.kv.pages_held() == 7


def test_truncating_gives_pages_back_exactly_when_a_page_empties(gpu):  # paging.rs:115-140
    mir = Mirror(gpu, Mirror.SMALL, 300)
    mir.append(gpu, 200)
    assert mir.kv.pages_in_use() == 4
    for length, pages in ((193, 4), (192, 3), (129, 3), (128, 2), (65, 2), (64, 1), (1, 1), (0, 0)):
        mir.truncate(length)
        assert mir.kv.pages_in_use() == pages
        assert mir.kv.pages_held() == 4
    mir.append(gpu, 200)
    mir.check_every_kernel(gpu)
    assert mir.kv.pages_held() == 4


def test_memory_follows_the_live_tokens_and_not_the_capacity(gpu):  # paging.rs:142-167
    mir = Mirror(gpu, Mirror.SMALL, 8192)
    assert (mir.kv.pages_held(), mir.kv.bytes_held()) == (0, 0)
    page = Mirror.LAYERS * 2 * m.PAGE_TOKENS * 2 * 16 * 4
    slab = m.SLAB_PAGES * page
    assert (mir.kv.page_bytes(), mir.kv.slab_bytes()) == (page, slab)
    mir.append(gpu, 10)
    assert (mir.kv.pages_held(), mir.kv.bytes_held()) == (1, slab)
    mir.append(gpu, 54)
    assert mir.kv.pages_held() == 1
    mir.append(gpu, 1)
    assert (mir.kv.pages_held(), mir.kv.bytes_held()) == (2, slab)
    mir.append(gpu, 8 * m.PAGE_TOKENS - 65)
    assert (mir.kv.pages_held(), mir.kv.bytes_held()) == (8, slab)
    mir.append(gpu, 1)
    assert (mir.kv.pages_held(), mir.kv.bytes_held()) == (9, 2 * slab)
    mir.append(gpu, 1000)
    assert mir.kv.pages_held() == m.pages_for(8 * m.PAGE_TOKENS + 1001)
    assert mir.kv.bytes_held() == 3 * slab


def test_repeated_appends_and_rollbacks_stay_exact(gpu):  # paging.rs:169-197
    mir = Mirror(gpu, Mirror.SMALL, 400)
    mir.append(gpu, 50)
    state = 0x2545F4914F6CDD1D
    mask = (1 << 64) - 1
    for step in range(150):
        state ^= (state << 13) & mask
        state ^= state >> 7
        state ^= (state << 17) & mask
        grow = (state & 7) + 1
        back = min((state >> 8) & 7, grow)
        room = max(0, 400 - mir.kv.len() - 1)
        mir.append(gpu, min(grow, room))
        mir.truncate(max(0, mir.kv.len() - back))
        assert mir.kv.pages_in_use() == m.pages_for(mir.kv.len())
        if step % 7 == 0:
            mir.check(gpu, 1 if step % 2 == 0 else 3)
        if mir.kv.len() > 330:
            mir.truncate(60)


def test_a_failed_write_keeps_no_pages_and_attention_refuses_unmapped_pages(gpu):  # paging.rs:199-216
    kv = m.DeviceKv(gpu, 1, Mirror.SMALL, 100, m.KvFormat.F32)
    too_many = gpu.zeros(101 * 32)
    with pytest.raises(m.Shape):
        kv.write(gpu, 0, too_many, too_many)
    assert (kv.pages_in_use(), kv.pages_held()) == (0, 0)
    kv.advance(70)
    for tokens in (1, 2, 12):
        with pytest.raises(m.HipError):
            gpu.attention(gpu.zeros(tokens * 4 * 16), kv, 0, 4, tokens, gpu.zeros(tokens * 4 * 16))


def test_a_capacity_that_is_not_a_page_multiple_fills_exactly(gpu):  # paging.rs:218-232
    mir = Mirror(gpu, Mirror.SMALL, 130)
    mir.append(gpu, 129)
    mir.check(gpu, 1)
    mir.append(gpu, 1)
    assert (mir.kv.len(), mir.kv.pages_in_use()) == (130, 3)
    extra = gpu.zeros(32)
    with pytest.raises(m.Shape):
        mir.kv.write(gpu, 0, extra, extra)
    with pytest.raises(m.Shape):
        mir.kv.advance(1)


def test_two_sequences_do_not_see_each_others_pages(gpu):  # paging.rs:234-256
    a = Mirror(gpu, Mirror.SMALL, 300)
    b = Mirror(gpu, Mirror.SMALL, 300)
    for rnd in range(6):
        a.append(gpu, 37)
        b.append(gpu, 45)
        if rnd % 2 == 1:
            a.truncate(max(0, a.kv.len() - 50))
        a.check(gpu, 1)
        b.check(gpu, 3)


@pytest.mark.parametrize("fmt", [m.KvFormat.F16, m.KvFormat.BF16])
def test_half_formats_round_on_store_and_attend_in_f32(gpu, fmt):  # kv_formats.rs
    for total in (1, 64, 65, 300):
        mir = Mirror(gpu, (8, 2, 128), 400, fmt)
        mir.append(gpu, total)
        mir.check_every_kernel(gpu)


@pytest.mark.parametrize("batch,lo,hi", [(4, 1, 700), (16, 512, 8193)])
def test_batched_paged_attention_over_a_shuffled_shared_pool(gpu, batch, lo, hi):
    """Config 2: 32 Q / 8 KV heads, head_dim 128, 16-token pages, ragged contexts, shuffled page tables from one pool;
    bf16 in and out, against the f64 reference of each sequence (max relative 1e-2). At its own size (batch 16,
    contexts uniform in [512, 8192], the longest pinned to 8192 and the shortest to 512) the longest sequences are
    split into more chunks than one merge level takes; the small case adds a one-position context."""
    print(f"case batch={batch} ctx in [{lo}, {hi})", flush=True)
    rng = np.random.default_rng(5 + batch)
    heads, kvh, hd, pt = 32, 8, 128, 16
    ctx = rng.integers(lo, hi, size=batch).astype(np.uint32)
    if lo == 1:
        ctx[0] = 1
    else:
        ctx[0], ctx[-1] = hi - 1, lo
    pages_each = [-(-int(c) // pt) for c in ctx]
    total = sum(pages_each)
    perm = rng.permutation(total)
    pool = m.PagePool(gpu, total, pt, kvh, hd, m.KvFormat.BF16)
    stride = max(pages_each)
    tables = np.zeros((batch, stride), np.uint32)
    keys, vals = [], []
    at = 0
    for b in range(batch):
        k = o.f32_to_bf16_rne(rng.standard_normal((pages_each[b] * pt, kvh, hd)).astype(np.float32))
        v = o.f32_to_bf16_rne(rng.standard_normal((pages_each[b] * pt, kvh, hd)).astype(np.float32))
        keys.append(o.bf16_to_f32(k)[:ctx[b]])
        vals.append(o.bf16_to_f32(v)[:ctx[b]])
        for i in range(pages_each[b]):
            pid = int(perm[at])
            at += 1
            tables[b, i] = pid
            page = np.concatenate([k[i * pt:(i + 1) * pt].transpose(1, 0, 2).ravel(),
                                   v[i * pt:(i + 1) * pt].transpose(1, 0, 2).ravel()])
            pool.write_page(pid, page)
    q = o.f32_to_bf16_rne(rng.standard_normal((batch, heads, hd)).astype(np.float32))
    out = gpu.typed(1, batch * heads * hd)
    pool.attention(gpu.typed(1, host=q), tables, ctx, heads, out)
    got = o.bf16_to_f32(gpu.download_typed(out)).reshape(batch, heads * hd)
    qf = o.bf16_to_f32(q).reshape(batch, heads * hd)
    for b in range(batch):
        exp = reference_attention(qf[b], keys[b].ravel(), vals[b].ravel(), heads, kvh, hd, int(ctx[b]) - 1, 1)
        rel = np.abs(got[b] - exp).max() / np.abs(exp).max()
        assert rel <= 1e-2, (b, rel)
