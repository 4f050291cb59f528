"""Counter-hash keys: known answers and structure (CPU).

Known answers are the reference's (tests/test_rng_streams.py:41-66); each is
checked against both oracles and against the product's host entry points
(sr_update_key / sr_state_key of the C ABI, the same source the kernels use).
"""

from __future__ import annotations

import pytest

from oracle import c_oracle, sr_oracle

UPDATE_KATS = [
    (0, 0, 0, 0x0EAA7511),
    (0, 1, 0, 0x7D2B5EA8),
    (42, 17, 9, 0xFA76534D),
    (0x12345678ABCDEFFE, 0xFEDCBA9876543210, 0xA5A5A5A5, 0xF820C188),
    (-1, 1 << 32, 1, 0x03D350C7),
]
STATE_KATS = [
    (0, 0, 0),
    (0, 1, 0x688990C0),
    (1, 0, 0x688990C0),
    (0x89ABCDEF, 1, 0x575E21BD),
    (0xFFFFFFFF, 2, 0x5681FFD9),
]
SEED = 0xFEDCBA9876543210


def _mask64(x):
    return x & 0xFFFFFFFFFFFFFFFF


@pytest.mark.parametrize("seed,step,index,expected", UPDATE_KATS)
def test_update_key_known_answers(seed, step, index, expected):
    import sr_states

    assert sr_oracle.update_key(seed, step, index) == expected
    assert c_oracle.lib().oc_update_key(_mask64(seed), _mask64(step), index & 0xFFFFFFFF) == expected
    assert sr_states.update_key(seed, step, index) == expected


@pytest.mark.parametrize("key,index,expected", STATE_KATS)
def test_state_key_known_answers(key, index, expected):
    import sr_states

    assert sr_oracle.state_key(key, index) == expected
    assert c_oracle.lib().oc_state_key(key, index) == expected
    assert sr_states.state_key(key, index) == expected


def test_h32_is_the_murmur3_finalizer_on_small_inputs():
    """Independent restatement: h32 equals fmix32 with the reference's constants."""

    def fmix(x):
        x ^= x >> 16
        x = (x * 0x7FEB352D) % 2**32
        x ^= x >> 15
        x = (x * 0x846CA68B) % 2**32
        return x ^ (x >> 16)

    for value in list(range(300)) + [2**31, 2**32 - 1, 0xDEADBEEF]:
        assert sr_oracle.h32(value) == fmix(value) == c_oracle.lib().oc_hash(value)
    # h32 is a bijection: inverting each step recovers the input.
    inv1, inv2 = pow(0x7FEB352D, -1, 2**32), pow(0x846CA68B, -1, 2**32)

    def unshift(x, s):
        y = x
        for _ in range(32 // s + 1):
            y = x ^ (y >> s)
        return y

    for value in (0, 1, 12345, 2**32 - 1, 0x9E3779B9):
        x = sr_oracle.h32(value)
        x = unshift(x, 16)
        x = (x * inv2) % 2**32
        x = unshift(x, 15)
        x = (x * inv1) % 2**32
        assert unshift(x, 16) == value


def test_changing_one_key_word_changes_the_key():
    """tests/test_rng_streams.py:69-78."""
    import sr_states

    seed, step, index = SEED, 0x123456789ABCDEF0, 13
    original = sr_states.update_key(seed, step, index)
    for bit in range(64):
        assert sr_states.update_key(seed ^ (1 << bit), step, index) != original
        assert sr_states.update_key(seed, step ^ (1 << bit), index) != original
    for bit in range(32):
        assert sr_states.update_key(seed, step, index ^ (1 << bit)) != original
    assert sr_states.update_key(seed + (1 << 64), step + (1 << 64), index) == original
    assert len({sr_states.state_key(original, i) for i in range(3)}) == 3


def test_sampled_update_keys_are_distinct():
    """tests/test_rng_streams.py:81-83, and the product agrees with the oracle."""
    import sr_states

    keys = {sr_states.update_key(42, step, index) for step in range(1, 1001) for index in range(120)}
    assert len(keys) == 120_000
    for step, index in [(1, 0), (999, 119), (2**40, 7)]:
        assert sr_states.update_key(42, step, index) == sr_oracle.update_key(42, step, index)


@pytest.mark.parametrize("value", [0, 1, 16, -1, 2**31, 2**63 + 7, 2**90 + 2**33 + 4])
def test_seeds_and_steps_use_their_low_64_bits(value):
    """tests/test_multi_tensor_tables.py:178-182: the kernel takes the low 64 bits."""
    import sr_states

    low = value % 2**64
    assert sr_states.update_key(value, value, 3) == sr_states.update_key(low, low, 3)
    assert sr_states._lib.low64(value) == low
