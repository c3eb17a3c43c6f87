"""Capacity buckets of the graph decoder pool: the reference's bucket rule and its cases
(assistant/backends.py:162-167; assistant/test_assistant.py:195-204), and the pool's guards.
Host logic only: no GPU is touched."""

import pytest
import torch

from efficientgpt_amd.fast_decode import GRAPH_BUCKETS, MAX_GRAPH_DECODERS, DecoderPool, pick_bucket


def test_reference_buckets_and_pool_size():
    assert GRAPH_BUCKETS == (256, 384, 512, 1024, 2048, 4096)
    assert MAX_GRAPH_DECODERS == 3


def test_pick_bucket_reference_cases():
    b = GRAPH_BUCKETS
    assert pick_bucket(317, b, 4096) == 384
    assert pick_bucket(384, b, 4096) == 384
    assert pick_bucket(385, b, 4096) == 512
    assert pick_bucket(1, b, 4096) == 256
    assert pick_bucket(4096, b, 4096) == 4096
    assert pick_bucket(4097, b, 4096) is None
    assert pick_bucket(600, b, 1000) == 1000  # a limit below the next bucket is still usable


def test_pick_bucket_against_brute_force():
    # the smallest allowed capacity (buckets at or under the limit, and the limit) that holds the request
    for buckets in ((64, 128, 256), (100,), (8, 4096, 16)):
        for limit in (1, 50, 100, 128, 300, 5000):
            allowed = sorted({x for x in buckets if x <= limit} | {limit})
            for need in range(0, 5200, 7):
                fits = [c for c in allowed if c >= need]
                assert pick_bucket(need, buckets, limit) == (fits[0] if fits else None), (buckets, limit, need)


def test_pool_guards_on_the_host():
    pool = DecoderPool(None, limit=1000)
    assert pool.capacity_for(300) == 384
    assert pool.capacity_for(999) == 1000
    with pytest.raises(ValueError):
        pool.capacity_for(1001)
    with pytest.raises(ValueError):
        pool.generate(torch.zeros((2, 4), dtype=torch.long), 4)
    with pytest.raises(ValueError):
        pool.generate(torch.zeros((1, 4), dtype=torch.long), 0)
    with pytest.raises(ValueError):
        DecoderPool(None, limit=0)
    with pytest.raises(ValueError):
        DecoderPool(None, max_decoders=0)
