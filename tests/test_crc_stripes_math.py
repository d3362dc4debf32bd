"""The CRC32C kernel's stripe decomposition on the CPU, against the oracle's CRC32C.

The CRC32C kernels give each stripe of a record to one wave: the stripe is
``groups`` groups of 1 KiB, lane l folds the 16-byte word at l * 16 of every
group as one slicing-by-4 chain of 4 dwords, and the lane keeps 8 chains,
chain c taking the stripe's groups c, c + 8, ... (counted from its first
group of record bytes), each advanced by shift(s, 8 * 1024 - 16) before its
next word.  At the end the chains are combined by Horner's rule in the order
of their last groups (shift(s, 1024) between them), each lane's register is
shifted past the lanes after it (x^(8 * 16 * (63 - l))), and the wave's XOR
is the stripe's raw CRC.  The first stripe is padded in front with zero bytes
and its whole groups of padding are skipped.  Stripe j is then shifted past
the stripes after it with the powers x^(8 * stripe_bytes * 2^i) (in the
workgroup, or by the combine kernel) and the initial value's term is added.

This replays that scheme in Python with the kernel's own tables (slicing,
advance, chain and lane shifts), over the stripe plans the library picks, and
checks every record's CRC32C against the oracle's (the reference's
kvsnap_crc32c_extend, csrc/dataplane/io.cpp:39-44); a variant that combines
the chains in the wrong order must fail.
"""
import random

import pytest

import oracle
from tests.test_checked_crc_math import gf_mul, xpow8n

RUN, CHAINS, LANES = 16, 8, 64
GROUP = LANES * RUN
MAX_STRIPES, RESIDENT_WAVES = 64, 256 * 16


def slicing_tables():
    return [[gf_mul(xpow8n(4 - i), v) for v in range(256)] for i in range(4)]


S = slicing_tables()
ADVANCE = xpow8n(CHAINS * GROUP - RUN)
G = [[gf_mul(ADVANCE, v << (8 * k)) for v in range(256)] for k in range(4)]
BEHIND = xpow8n(GROUP)
H = [[gf_mul(BEHIND, v << (8 * k)) for v in range(256)] for k in range(4)]
M = [xpow8n(RUN * (63 - lane)) for lane in range(LANES)]


def lookup(tables, x):
    return tables[0][x & 0xFF] ^ tables[1][(x >> 8) & 0xFF] ^ tables[2][(x >> 16) & 0xFF] ^ tables[3][x >> 24]


def chain(state, run):
    for k in range(0, RUN, 4):
        state = lookup(S, state ^ int.from_bytes(run[k:k + 4], "little"))
    return state


def plan(record_bytes, n_records, max_partials=0):
    """The library's stripe plan (crc_plan in kernels.hip)."""
    total = max(1, -(-record_bytes // GROUP))
    n = max(1, n_records)
    cap = MAX_STRIPES if not max_partials else min(MAX_STRIPES, max(1, max_partials // n))
    cap = min(cap, total)
    best, chosen = None, (total, 1)
    for s in range(1, cap + 1):
        g = -(-total // s)
        stripes = -(-total // g)
        cost = -(-(n * stripes) // RESIDENT_WAVES) * (g + 2)
        if best is None or cost < best:
            best, chosen = cost, (g, stripes)
    groups, stripes = chosen
    return groups, stripes, stripes * groups * GROUP - record_bytes


def stripe_raw(record, start, groups, wrong_order=False):
    """One wave's job: the raw CRC of the stripe whose first byte is at record offset ``start``."""
    lead = (-start) // GROUP if start < 0 else 0

    def run(g, lane):
        at = start + g * GROUP + lane * RUN
        if at >= 0:
            return bytes(record[at:at + RUN])
        return bytes(record[0:max(at + RUN, 0)]).rjust(RUN, b"\0")     # front padding reads as zeros

    total = 0
    m = groups - lead
    for lane in range(LANES):
        acc = [0] * CHAINS
        for g in range(lead, groups):
            c = (g - lead) % CHAINS
            acc[c] = chain(lookup(G, acc[c]), run(g, lane))
        x = 0
        order = range(CHAINS - 1, -1, -1) if not wrong_order else range(CHAINS)
        for i, d in enumerate(order):
            pick = acc[(m - 1 - d) % CHAINS]
            x = (0 if i == 0 else lookup(H, x)) ^ pick
        total ^= gf_mul(M[lane], x)
    return total


def record_crc(record, groups, stripes, pad, prior=0, **variant):
    stripe_bytes = groups * GROUP
    powers = [xpow8n(stripe_bytes << i) for i in range(6)]
    x = 0
    for j in range(stripes):
        part = stripe_raw(record, j * stripe_bytes - pad, groups, **variant)
        for i in range(6):
            if ((stripes - 1 - j) >> i) & 1:
                part = gf_mul(powers[i], part)
        x ^= part
    init_term = gf_mul(xpow8n(len(record)), prior ^ 0xFFFFFFFF)
    return (init_term ^ x) ^ 0xFFFFFFFF


@pytest.mark.parametrize("record_bytes,n_records", [
    (64, 1), (1024, 1), (1040, 2), (12288, 3), (20480, 4096), (17408, 8192), (9216, 40000), (0, 1),
])
def test_the_stripe_scheme_gives_the_oracle_crc32c(record_bytes, n_records):
    groups, stripes, pad = plan(record_bytes, n_records)
    assert 1 <= stripes <= MAX_STRIPES and (0 <= pad < groups * GROUP or record_bytes == 0)
    rng = random.Random(record_bytes + n_records)
    record = bytes(rng.getrandbits(8) for _ in range(record_bytes))
    prior = rng.getrandbits(32)
    assert record_crc(record, groups, stripes, pad, prior) == oracle.crc32c(record, prior)


def test_plans_with_padding_skip_whole_groups_and_split_lanes_across_the_record_start():
    # 3 groups over 2 stripes of 2 groups: stripe 0 is one whole group of padding (skipped), then a
    # group of record bytes; 5 groups over 2 stripes of 3: a partial first group; 19 groups in one
    # stripe of 20 (a partial batch of chains after the first whole one).
    rng = random.Random(5)
    for record_bytes, groups, stripes in [(3 * GROUP, 2, 2), (5 * GROUP - 1000, 3, 2), (GROUP + 16, 1, 2),
                                          (19 * GROUP + 48, 20, 1)]:
        pad = stripes * groups * GROUP - record_bytes
        record = bytes(rng.getrandbits(8) for _ in range(record_bytes))
        assert record_crc(record, groups, stripes, pad) == oracle.crc32c(record)


def test_the_plan_fills_the_chip_with_one_round_for_the_8k_session():
    # 512 Qwen3-8B records of 2,359,296 bytes: 8 stripes of 288 groups, 4096 jobs (one per resident wave).
    assert plan(2359296, 512) == (288, 8, 0)
    # A tensor-parallel rank's shard (TP = 8): 294,912-byte records, 8 stripes of 36 groups.
    assert plan(294912, 512) == (36, 8, 0)
    # A workspace bound caps the stripes (the no-allocation entry point's 65536 partials).
    groups, stripes, _ = plan(2359296, 16384, max_partials=65536)
    assert stripes * 16384 <= 65536


def test_a_scheme_that_combines_the_chains_in_the_wrong_order_fails():
    rng = random.Random(9)
    record = bytes(rng.getrandbits(8) for _ in range(11 * GROUP))
    groups, stripes, pad = 11, 1, 0
    assert record_crc(record, groups, stripes, pad) == oracle.crc32c(record)
    assert record_crc(record, groups, stripes, pad, wrong_order=True) != oracle.crc32c(record)
