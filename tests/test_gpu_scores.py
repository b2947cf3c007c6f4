"""GPU parity: paged chunk scores (ds_chunk_scores).

Mirrors the reference's device tests (tests/test_retrieval_npu.py:36-85 and
tests/test_retrieval_dynamic_npu.py:15-45): a dense GQA softmax reference with
reordered pages and partial chunks (rtol 1e-3, atol 1e-6), and zero keys,
whose uniform softmax gives exactly 1/L per chunk.  Without a supplied LSE
(softmax_lse=None, the reference's chunk_attention_scores default,
diffspec/runtime.py:321-322) the same checks run against the oracle's
per-row logsumexp.
"""

import pytest
import torch

from helpers import O, assert_scores_close, default_scale, gen, lse_for, paged_keys, randn, uniform_lengths

pytestmark = pytest.mark.gpu


def _gpu_scores(query, key_cache, lse, table, lengths, chunk, scale, device, head_reduce="mean"):
    from ds355.kernels import paged_chunk_attention_scores

    return paged_chunk_attention_scores(
        query.to(device), key_cache.to(device), None if lse is None else lse.to(device), table.to(device),
        torch.tensor(lengths, dtype=torch.int32, device=device),
        chunk_size=chunk, max_seq_len=max(lengths), scale=scale, head_reduce=head_reduce,
    ).cpu()


@pytest.mark.parametrize("block_size", [64, 1024, 1536])
@pytest.mark.parametrize("num_query_heads,num_kv_heads", [(4, 1), (8, 2), (6, 1), (12, 2)])
@pytest.mark.parametrize("chunk_size", [16, 64])
def test_paged_scores_match_dense_bf16_gqa(cuda, block_size, num_query_heads, num_kv_heads, chunk_size):
    torch.manual_seed(123)
    head_dim = 256
    lengths = [2 * block_size + 13, block_size + 25]
    query = torch.randn((2, num_query_heads, head_dim), dtype=torch.bfloat16)
    keys = torch.randn((9, block_size, num_kv_heads, head_dim), dtype=torch.bfloat16)
    tables = torch.tensor([[4, 1, 7], [8, 2, 5]], dtype=torch.int32)
    scale = head_dim ** -0.5
    references, normalizers = [], []
    max_chunks = (max(lengths) + chunk_size - 1) // chunk_size
    for row, length in enumerate(lengths):
        dense_keys = keys[tables[row].long()].reshape(-1, num_kv_heads, head_dim)[:length]
        grouped = query[row].float().reshape(num_kv_heads, -1, head_dim)
        logits = torch.einsum("hgd,thd->hgt", grouped, dense_keys.float()).reshape(num_query_heads, length) * scale
        normalizers.append(torch.logsumexp(logits, dim=-1))
        probabilities = logits.softmax(-1)
        reference = torch.zeros(max_chunks)
        for chunk in range((length + chunk_size - 1) // chunk_size):
            reference[chunk] = probabilities[:, chunk * chunk_size:(chunk + 1) * chunk_size].mean()
        references.append(reference)
    actual = _gpu_scores(query, keys, torch.stack(normalizers), tables, lengths, chunk_size, scale, cuda)
    assert_scores_close(actual, torch.stack(references))
    assert torch.isfinite(actual).all()
    oracle = O.paged_chunk_attention_scores(query, keys, torch.stack(normalizers), tables,
                                            torch.tensor(lengths), chunk_size=chunk_size,
                                            max_seq_len=max(lengths), scale=scale)
    assert_scores_close(actual, oracle)


def test_zero_keys_give_uniform_mass(cuda):
    query = torch.ones((2, 4, 256), dtype=torch.bfloat16)
    keys = torch.zeros((9, 1024, 1, 256), dtype=torch.bfloat16)
    table = torch.tensor([[4, 1, 7], [8, 2, 5]], dtype=torch.int32)
    for chunks in [1, *range(9, 19)]:
        lengths = [16 * chunks - 3, min(100, 16 * chunks - 3)]
        lse = torch.tensor(lengths, dtype=torch.float32).log()[:, None].expand(-1, 4).contiguous()
        actual = _gpu_scores(query, keys, lse, table, lengths, 16, 256 ** -0.5, cuda)
        expected = torch.zeros((2, chunks))
        for row, length in enumerate(lengths):
            expected[row, : (length + 15) // 16] = 1.0 / length
        assert_scores_close(actual, expected)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim,chunk,block_size", [(128, 64, 128), (64, 32, 16), (128, 128, 256), (96, 48, 64),
                                                       (64, 48, 64), (128, 64, 40), (64, 32, 8)])
def test_ragged_batch_matches_oracle(cuda, dtype, head_dim, chunk, block_size):
    g = gen(3)
    hq, hkv = 32, 4
    lengths = uniform_lengths(9, 1, 5000, g) + [0, 1, chunk, chunk + 1]
    query = randn((len(lengths), hq, head_dim), dtype, g)
    key_cache, table = paged_keys(lengths, hkv, head_dim, block_size, dtype, g)
    scale = default_scale(head_dim)
    lse = lse_for(query, key_cache, table, lengths, scale)
    actual = _gpu_scores(query, key_cache, lse, table, lengths, chunk, scale, cuda)
    expected = O.paged_chunk_attention_scores(query, key_cache, lse, table, torch.tensor(lengths), chunk_size=chunk,
                                              max_seq_len=max(lengths), scale=scale)
    assert_scores_close(actual, expected)


@pytest.mark.parametrize("head_dim,chunk,block_size,dtype", [
    (128, 64, 64, torch.bfloat16),
    (64, 32, 40, torch.float16),     # pages looked up per lane
    (256, 128, 48, torch.bfloat16),  # pages by division, wide heads
])
def test_head_reduce_max_matches_oracle(cuda, head_dim, chunk, block_size, dtype):
    g = gen(4)
    lengths = [3000, 777, 64, chunk + 1]
    query = randn((len(lengths), 32, head_dim), dtype, g)
    key_cache, table = paged_keys(lengths, 4, head_dim, block_size, dtype, g)
    scale = default_scale(head_dim)
    lse = lse_for(query, key_cache, table, lengths, scale)
    actual = _gpu_scores(query, key_cache, lse, table, lengths, chunk, scale, cuda, head_reduce="max")
    expected = O.paged_chunk_attention_scores(query, key_cache, lse, table, torch.tensor(lengths), chunk_size=chunk,
                                              max_seq_len=max(lengths), scale=scale, head_reduce="max")
    assert_scores_close(actual, expected)


def test_headline_shape_scores(cuda):
    """16 requests, L ~ U[4096, 40960], 32 q heads / 4 KV heads x 128, chunk 64."""
    g = gen(0)
    lengths = uniform_lengths(16, 4096, 40960, g)
    query = randn((16, 32, 128), torch.bfloat16, g)
    key_cache, table = paged_keys(lengths, 4, 128, 128, torch.bfloat16, g)
    scale = default_scale(128)
    lse = lse_for(query, key_cache, table, lengths, scale)
    actual = _gpu_scores(query, key_cache, lse, table, lengths, 64, scale, cuda)
    expected = O.paged_chunk_attention_scores(query, key_cache, lse, table, torch.tensor(lengths), chunk_size=64,
                                              max_seq_len=max(lengths), scale=scale)
    assert_scores_close(actual, expected)
    # Size-independent property: the chunk masses of a row, weighted by the
    # chunk sizes, sum to 1 (a softmax with the exact LSE).
    for b, n in enumerate(lengths):
        c = (n + 63) // 64
        sizes = torch.full((c,), 64.0)
        sizes[-1] = n - (c - 1) * 64
        assert abs(float((actual[b, :c].double() * sizes.double()).sum()) - 1.0) < 2e-3


def test_reference_validation_messages(cuda):
    from ds355.kernels import paged_chunk_attention_scores

    q = torch.zeros((2, 4, 64), dtype=torch.bfloat16, device=cuda)
    k = torch.zeros((3, 16, 2, 64), dtype=torch.bfloat16, device=cuda)
    bt = torch.zeros((2, 3), dtype=torch.int32, device=cuda)
    sl = torch.ones(2, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="softmax_lse must contain one value per query head"):
        paged_chunk_attention_scores(q, k, torch.zeros(3, device=cuda), bt, sl, chunk_size=4, max_seq_len=4, scale=1.0)
    with pytest.raises(ValueError, match="query heads must be divisible by KV heads"):
        paged_chunk_attention_scores(q[:, :3], k, torch.zeros(6, device=cuda), bt, sl, chunk_size=4, max_seq_len=4,
                                     scale=1.0)
    with pytest.raises(ValueError, match=r"query must have shape"):
        paged_chunk_attention_scores(q[0], k, torch.zeros(8, device=cuda), bt, sl, chunk_size=4, max_seq_len=4, scale=1.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim,chunk,block_size", [(128, 64, 128), (64, 32, 16), (128, 128, 256), (96, 48, 64),
                                                       (256, 16, 1024), (64, 48, 64), (128, 64, 40)])
@pytest.mark.parametrize("hq,hkv", [(32, 4), (12, 2), (16, 1), (12, 4)])
def test_lse_free_ragged_batch_matches_oracle(cuda, dtype, head_dim, chunk, block_size, hq, hkv):
    g = gen(11)
    lengths = uniform_lengths(7, 1, 5000, g) + [0, 1, chunk, chunk + 1]
    query = randn((len(lengths), hq, head_dim), dtype, g)
    key_cache, table = paged_keys(lengths, hkv, head_dim, block_size, dtype, g)
    scale = default_scale(head_dim)
    actual = _gpu_scores(query, key_cache, None, table, lengths, chunk, scale, cuda)
    expected = O.paged_chunk_attention_scores(query, key_cache, None, table, torch.tensor(lengths), chunk_size=chunk,
                                              max_seq_len=max(lengths), scale=scale)
    assert_scores_close(actual, expected)
    # The same scores as with the exact LSE supplied.
    lse = lse_for(query, key_cache, table, lengths, scale)
    supplied = _gpu_scores(query, key_cache, lse, table, lengths, chunk, scale, cuda)
    assert_scores_close(actual, supplied)


def test_lse_free_zero_keys_give_uniform_mass(cuda):
    query = torch.ones((2, 4, 256), dtype=torch.bfloat16)
    keys = torch.zeros((9, 1024, 1, 256), dtype=torch.bfloat16)
    table = torch.tensor([[4, 1, 7], [8, 2, 5]], dtype=torch.int32)
    for chunks in [1, 9, 64, 192]:
        lengths = [16 * chunks - 3, min(100, 16 * chunks - 3)]
        actual = _gpu_scores(query, keys, None, table, lengths, 16, 256 ** -0.5, cuda)
        expected = torch.zeros((2, chunks))
        for row, length in enumerate(lengths):
            expected[row, : (length + 15) // 16] = 1.0 / length
        assert_scores_close(actual, expected)


def test_lse_free_large_logits_stay_finite(cuda):
    """Logits in the hundreds: the running max keeps every 2^(x - m) in range."""
    g = gen(12)
    lengths = [4000, 333, 64]
    query = (randn((3, 32, 128), torch.bfloat16, g).float() * 4).to(torch.bfloat16)
    key_cache, table = paged_keys(lengths, 4, 128, 64, torch.bfloat16, g)
    scale = 1.0
    actual = _gpu_scores(query, key_cache, None, table, lengths, 64, scale, cuda)
    assert torch.isfinite(actual).all()
    expected = O.paged_chunk_attention_scores(query, key_cache, None, table, torch.tensor(lengths), chunk_size=64,
                                              max_seq_len=max(lengths), scale=scale)
    assert_scores_close(actual, expected)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (12, 2), (16, 1), (6, 6)])
def test_lse_free_long_rows_take_wider_slices(cuda, hq, hkv):
    """Rows of up to 2500 chunks: a (row, KV head) finalizes in at most 8 workgroups, so each
    takes slices wider than its 256 threads (chunks t and t + 256 of the slice).  Past 1024
    chunks per row the LSE merge loads two heads' pairs at once: groups of 4 and 16 heads
    (2 and 8 lane phases), 6 (3 phases, one block of lanes each) and 1 (one head per load)."""
    g = gen(13)
    lengths = [40000, 23000, 17, 4097, 16 * 1024 + 1]
    query = randn((len(lengths), hq, 64), torch.bfloat16, g)
    key_cache, table = paged_keys(lengths, hkv, 64, 256, torch.bfloat16, g)
    scale = default_scale(64)
    actual = _gpu_scores(query, key_cache, None, table, lengths, 16, scale, cuda)
    expected = O.paged_chunk_attention_scores(query, key_cache, None, table, torch.tensor(lengths), chunk_size=16,
                                              max_seq_len=max(lengths), scale=scale)
    assert_scores_close(actual, expected)
    lse = lse_for(query, key_cache, table, lengths, scale)
    supplied = _gpu_scores(query, key_cache, lse, table, lengths, 16, scale, cuda)
    assert_scores_close(actual, supplied)
    for b, n in enumerate(lengths):  # a row's chunk masses add up to one
        c = (n + 15) // 16
        sizes = torch.full((c,), 16.0)
        sizes[-1] = n - (c - 1) * 16
        assert abs(float((actual[b, :c].double() * sizes.double()).sum()) - 1.0) < 2e-3


def test_lse_free_headline_shape_scores(cuda):
    """16 requests, L ~ U[4096, 40960], 32 q heads / 4 KV heads x 128, chunk 64, no LSE."""
    g = gen(0)
    lengths = uniform_lengths(16, 4096, 40960, g)
    query = randn((16, 32, 128), torch.bfloat16, g)
    key_cache, table = paged_keys(lengths, 4, 128, 128, torch.bfloat16, g)
    scale = default_scale(128)
    actual = _gpu_scores(query, key_cache, None, table, lengths, 64, scale, cuda)
    expected = O.paged_chunk_attention_scores(query, key_cache, None, table, torch.tensor(lengths), chunk_size=64,
                                              max_seq_len=max(lengths), scale=scale)
    assert_scores_close(actual, expected)
    for b, n in enumerate(lengths):
        c = (n + 63) // 64
        sizes = torch.full((c,), 64.0)
        sizes[-1] = n - (c - 1) * 64
        assert abs(float((actual[b, :c].double() * sizes.double()).sum()) - 1.0) < 2e-3
