"""The Q8_0 row kernels split a flat block number into (row, block in row)
with a float reciprocal estimate corrected by one step (codec.hip,
row_block). Emulated here in float32 / uint32 arithmetic and checked against
exact division, including rows of 2^24 blocks and more, where 24-bit
multiplies would drop the high bits of the row length."""
import numpy as np


def _umul24(a, b):
    return np.uint32((int(a) & 0xFFFFFF) * (int(b) & 0xFFFFFF) & 0xFFFFFFFF)


def _row_block(t, bpr, use24):
    inv = np.float32(1.0) / np.float32(bpr)
    q = int(np.float32(t) * inv)
    mul = (lambda a, b: int(_umul24(a, b))) if use24 else (lambda a, b: (a * b) & 0xFFFFFFFF)
    if mul(q, bpr) > t:
        q -= 1
    if mul(q + 1, bpr) <= t:
        q += 1
    return q, (t - mul(q, bpr)) & 0xFFFFFFFF


def _device_row_block(t, bpr):
    # The kernel's rule: 24-bit multiplies only while bpr < 2^24.
    return _row_block(t, bpr, bpr < (1 << 24))


def test_row_split_matches_division():
    rng = np.random.default_rng(3)
    bprs = [1, 2, 3, 18, 64, 1000, (1 << 24) - 1, 1 << 24, (1 << 24) + 1000, (1 << 27) - 3, 1 << 27]
    for bpr in bprs:
        # t = blk0 + k with blk0 < bpr and k < 1024 (a tile's blocks).
        for _ in range(200):
            blk0 = int(rng.integers(0, bpr))
            k = int(rng.integers(0, 1024))
            t = blk0 + k
            assert _device_row_block(t, bpr) == divmod(t, bpr), (t, bpr)
        for t in (0, bpr - 1, bpr, bpr + 1023, 2 * bpr - 1 if bpr < 1024 else bpr + 999):
            assert _device_row_block(t, bpr) == divmod(t, bpr), (t, bpr)


def test_24_bit_split_fails_past_2_pow_24_blocks():
    """The case the 32-bit branch exists for: one row of 2^29 + 32,000 values
    (2^24 + 1,000 blocks); block 1,000 + 2^24 - 1 of row 0 would map to row 1
    with 24-bit multiplies."""
    bpr = (1 << 24) + 1000
    t = bpr - 1
    assert _row_block(t, bpr, True) != divmod(t, bpr)
    assert _device_row_block(t, bpr) == divmod(t, bpr)
