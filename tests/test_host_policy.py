"""Host policy of split-K attention (rosevine_amd/hip.py, restating runtime/src/hip.rs:481-497), on
the CPU: the chunk count and the partial scratch it needs."""
from rosevine_amd import hip


def test_scratch_bounds_every_chunk_count():
    # runtime/tests/hip_ops.rs:321-329, for the reference's target and for the MI355X one
    for target, scratch_target in ((hip.ATTN_TARGET_BLOCKS, hip.ATTN_TARGET_BLOCKS),
                                   (hip.ATTN_TARGET_BLOCKS_MI355X, hip.ATTN_TARGET_BLOCKS_MI355X)):
        for min_chunk in (hip.ATTN_MIN_CHUNK, 32):
            for n_tok in (1, 2, 3, 8, 31, 64, 256):
                for longest in (1, 63, 64, 65, 1000, 16_384, 262_144):
                    chunks = hip.attention_chunks(n_tok, 16, longest, target, min_chunk)
                    assert 1 <= chunks <= -(-longest // min_chunk)
                    assert n_tok * 16 * chunks * 514 <= hip.attention_split_scratch(n_tok, 16, 512, scratch_target)


def test_reference_case_table_chunk_counts():
    # the chunk column of runtime/tests/hip_ops.rs:273-299, which that test asserts for each case:
    # (queries, longest key range) -> chunks, 16 query heads, the reference's target
    cases = [(4, 1024, 16), (1, 5000, 64), (8, 5000, 8), (64, 5000, 1), (1, 3, 1), (1, 129, 3)]
    for n_tok, longest, want in cases:
        assert hip.attention_chunks(n_tok, 16, longest) == want, (n_tok, longest)


def test_mi355x_policy_for_the_bench_layers():
    # one token at depth 16384: a global layer's 16,385 keys in 128 chunks of 129 keys; a
    # sliding-window layer's 1024 keys in 32 chunks of 32 (one 32-key stage per workgroup)
    t, m = hip.ATTN_TARGET_BLOCKS_MI355X, 32
    assert hip.attention_chunks(1, 16, 16_385, t, m) == 128
    assert hip.attention_chunks(1, 16, 1024, t, m) == 32
    # the reference's minimum chunk keeps 16 chunks of 64 keys for the window
    assert hip.attention_chunks(1, 16, 1024, t) == 16
