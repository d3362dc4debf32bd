"""The CRC32C kernel's stripe decomposition on the CPU, against the oracle's CRC32C.

The CRC32C kernels give each stripe of a record to one wave: the stripe is
``groups`` groups of 1 KiB, lane l folds the 16-byte word at l * 16 of every
group, and the lane keeps 6 chains, chain c taking the stripe's groups c,
c + 6, ... (counted from its first group of record bytes):
acc' = shift(acc, 6 * 1024) ^ R(word), R the word's raw CRC from a zero
register in four slicing-by-4 steps.  At the end the chains are combined by Horner's rule in the order
of their last groups (shift(s, 1024) between them), each lane's register is
shifted past the lanes after it (x^(8 * 16 * (63 - l))), and the wave's XOR
is the stripe's raw CRC.  The first stripe is padded in front with zero bytes
and its whole groups of padding are skipped.  Stripe j is then shifted past
the stripes after it with the powers x^(8 * stripe_bytes * 2^i) (in the
workgroup, or by the combine kernel) and the initial value's term is added.

This replays that scheme in Python with the kernel's own tables (slicing,
advance by nibbles, chain and lane shifts), over the stripe plans the library
picks, and checks every record's CRC32C against the oracle's (the reference's
kvsnap_crc32c_extend, csrc/dataplane/io.cpp:39-44); a variant that combines
the chains in the wrong order must fail.  It also replays the kernel's LDS
addressing (v_perm_b32 byte moves into a per-lane column constant): every
lane's lookups of the private slicing and advance tables land in its own
bank and on the entry the fill put there.  And it replays the addresses the
aligned kernels' first batch loads (its one path with no branches, clamped):
every one is a word of the record, and every word folded is the stripe's own.
"""
import functools
import operator
import random

import pytest

import oracle
from tests.test_checked_crc_math import gf_mul, xpow8n

RUN, CHAINS, LANES = 16, 6, 64
GROUP = LANES * RUN
MAX_STRIPES, RESIDENT_WAVES = 64, 256 * 16


def slicing_tables():
    return [[gf_mul(xpow8n(4 - i), v) for v in range(256)] for i in range(4)]


S = slicing_tables()
ADVANCE = xpow8n(CHAINS * GROUP)
GN = [[gf_mul(ADVANCE, v << (4 * i)) for v in range(16)] for i in range(8)]     # the advance, by nibbles
BEHIND = xpow8n(GROUP)
H = [[gf_mul(BEHIND, v << (8 * k)) for v in range(256)] for k in range(4)]
M = [xpow8n(RUN * (63 - lane)) for lane in range(LANES)]


def lookup(tables, x):
    return tables[0][x & 0xFF] ^ tables[1][(x >> 8) & 0xFF] ^ tables[2][(x >> 16) & 0xFF] ^ tables[3][x >> 24]


def advance(x):
    return functools.reduce(operator.xor, (GN[i][(x >> (4 * i)) & 15] for i in range(8)))


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
            acc[c] = advance(acc[c]) ^ chain(0, run(g, lane))
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


# ---- the LDS layout of the private tables ------------------------------------------------------------

H_BYTES, GN_BYTES, S_BYTES = 4096, 16384, 131072
GN_AT, S_AT = H_BYTES, H_BYTES + GN_BYTES


def perm(x, cols, selector):
    """v_perm_b32(x, cols, selector): byte k of the result is byte (selector byte k) of {x: 7-4, cols: 3-0};
    selector 0x0C gives 0x00."""
    pool = cols.to_bytes(4, "little") + x.to_bytes(4, "little")
    out = 0
    for k in range(4):
        sel = (selector >> (8 * k)) & 0xFF
        out |= (0 if sel == 0x0C else pool[sel]) << (8 * k)
    return out


def columns(lane):
    col = (lane & 31) * 4
    return col | ((col + 128) << 8) | (1 << 16)


S_SELECTORS = (0x0C0C0400, 0x0C0C0501, 0x0C020600, 0x0C020701)
GN_LOOKUPS = [(page, half, 0x0C0C0000 | ((4 + page) << 8) | half) for page in range(4) for half in (0, 1)]


def fill_entry(chunk):
    """(table, v) of the S entry whose four lane columns the fill writes as 16-byte chunk `chunk`."""
    half, r = chunk >> 12, chunk & 4095
    return 2 * half + ((r >> 3) & 1), r >> 4


def filled_lds():
    """The bytes crc_fill_tables writes: {byte address: table word}."""
    lds = {}
    for k in range(8):                                  # S: thread t writes chunk k * 1024 + t
        for t in range(1024):
            chunk = k * 1024 + t
            table, v = fill_entry(chunk)
            for j in range(4):
                assert S_AT + 16 * chunk + 4 * j not in lds
                lds[S_AT + 16 * chunk + 4 * j] = S[table][v]
    for t in range(1024):
        e = t >> 3                                      # Gn entry e, four lane columns
        nib_table, nib = e >> 4, e & 15
        for k in range(4):
            lds[GN_AT + (nib_table >> 1) * 4096 + nib * 256 + (nib_table & 1) * 128 + (t & 7) * 16 + 4 * k] = \
                GN[nib_table][nib]
        lds[4 * t] = H[t >> 8][t & 255]
    return lds


def test_each_wave_write_of_the_s_fill_covers_one_kib_of_consecutive_banks():
    for k in range(8):
        for wave in range(16):
            chunks = [k * 1024 + 64 * wave + lane for lane in range(64)]
            assert chunks == list(range(chunks[0], chunks[0] + 64))      # 1 KiB contiguous
            assert {(4 * c + j) % 32 for c in chunks[:8] for j in range(4)} == set(range(32))  # 8 lanes, 32 banks


def test_the_private_tables_fill_the_lds_once_and_every_lane_reads_its_own_bank_and_entry():
    lds = filled_lds()
    assert len(lds) == (H_BYTES + GN_BYTES + S_BYTES) // 4 and max(lds) < H_BYTES + GN_BYTES + S_BYTES
    rng = random.Random(5)
    for lane in range(64):
        cols = columns(lane)
        for x in [0, 0xFFFFFFFF] + [rng.getrandbits(32) for _ in range(40)]:
            for i, selector in enumerate(S_SELECTORS):          # slicing-by-4 lookups, crc_step_all
                address = S_AT + perm(x, cols, selector)
                assert (address // 4) % 32 == lane % 32
                assert lds[address] == S[i][(x >> (8 * i)) & 0xFF]
            lo, hi = x & 0x0F0F0F0F, (x >> 4) & 0x0F0F0F0F       # the advance, crc_fold_batch
            found = 0
            for page, half, selector in GN_LOOKUPS:
                address = GN_AT + page * 4096 + perm(hi if half else lo, cols, selector)
                assert (address // 4) % 32 == lane % 32
                nibble = 2 * page + half
                assert lds[address] == GN[nibble][(x >> (4 * nibble)) & 15]
                found ^= lds[address]
            assert found == gf_mul(ADVANCE, x)


# ---------------------------------------------------------------- the aligned kernels' first-batch addresses


def first_batch_loads(start, groups, lane):
    """crc_stripe_first's loads (kernels.hip, aligned records): per chain, the record offset loaded.  A chain
    past the stripe's groups loads the batch's last group again, a word of front padding the record's first
    word (crc_first_words_kept zeroes both once they have landed)."""
    lead = (-start) // GROUP if start < 0 else 0
    count = min(CHAINS, groups - lead)
    at = start + lead * GROUP
    return lead, count, [max(at + min(c, count - 1) * GROUP + lane * RUN, 0) for c in range(CHAINS)]


@pytest.mark.parametrize("record_bytes,n_records", [
    (16, 1), (16, 300), (48, 7), (1040, 2), (1280, 29), (12000, 8192), (12288, 3), (17408, 5000), (20480, 4096),
    (294912, 512), (2359296, 512), (4096 * 1024 + 16, 3), (36 * 1024 * 9 + 16, 1000),
])
def test_the_aligned_first_batch_loads_only_record_words(record_bytes, n_records):
    """Every offset the aligned kernels' first batch loads (clamped chains included, for every stripe and
    lane) lies inside the record, and every word the batch folds (chains below its count, lanes past the
    padding) is the stripe's own."""
    groups, stripes, pad = plan(record_bytes, n_records)
    for j in range(stripes):
        start = j * groups * GROUP - pad
        for lane in range(LANES):
            lead, count, loads = first_batch_loads(start, groups, lane)
            assert count >= 1
            for off in loads:
                assert 0 <= off <= record_bytes - RUN, (record_bytes, j, lane, off)
            for c in range(count):
                word = start + (lead + c) * GROUP + lane * RUN
                if word >= 0:
                    assert loads[c] == word, (record_bytes, j, c, lane)
                else:
                    assert c == 0 and word > -GROUP     # only chain 0 can hold padding, less than a group


def test_an_unclamped_first_batch_would_load_outside_the_record():
    """The replay catches the mistake it guards against: without the clamp to the record's first word, a
    16-byte record's padding lanes would load before the record."""
    groups, stripes, pad = plan(16, 1)
    start = -pad
    lead = (-start) // GROUP
    assert min(start + lead * GROUP + lane * RUN for lane in range(LANES)) < 0
    assert all(first_batch_loads(start, groups, lane)[2][0] == 0 for lane in range(LANES - 1))
