"""Decode bucket policy of the graph helpers: the reference's own known
answers (tests/unit/test_step_executor.py:372-384)."""

from __future__ import annotations

import pytest

from kairyu_amd.graphs import bucket_for, decode_buckets


def test_decode_buckets_shape():
    assert decode_buckets(32) == (1, 2, 4, 8, 16, 24, 32)
    assert decode_buckets(48) == (1, 2, 4, 8, 16, 24, 32, 40, 48)
    assert decode_buckets(3) == (1, 2, 3)
    with pytest.raises(ValueError):
        decode_buckets(0)


def test_bucket_for():
    buckets = decode_buckets(32)
    assert bucket_for(1, buckets) == 1
    assert bucket_for(5, buckets) == 8
    assert bucket_for(32, buckets) == 32
    assert bucket_for(33, buckets) is None
