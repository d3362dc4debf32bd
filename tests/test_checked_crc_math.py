"""The checked restore's CRC32C decomposition on the CPU, against the oracle's CRC32C.

restore_checked_kernel gives each (block, span) job to one wave: lane l folds
the 16-byte slots l, l + 64, ... of its span, advancing its accumulator by one
1 KiB row per slot, then moves it to the span's end by x^(128 ((r - 1 - l) mod
64)) with r = slots mod 64; an 8-byte word past the slots is folded by lane 0
after the others move past it by x^64.  restore_checked_finish_kernel moves
each span's partial to the end of its record and adds the initial value's term.
This replays that scheme in Python, lane by lane, on spans of every length
class (whole rows, a short last row, fewer slots than lanes, an 8-byte word)
and checks the records' CRC32C against the oracle's (the reference's
kvsnap_crc32c_extend, csrc/dataplane/io.cpp:39-44), and that the shift a
whole-rows-only design would use fails on a short last row.
"""
import random

import oracle

POLY = 0x82F63B78


def gf_mul(a, b):
    """a * b mod P, reflected (bit 31 is x^0)."""
    p = 0
    for i in range(32):
        if (a >> (31 - i)) & 1:
            p ^= b
        b = (b >> 1) ^ (POLY if b & 1 else 0)
    return p


def xpow8n(n):
    """x^(8 n) mod P by squaring."""
    result, square, e = 0x80000000, 0x40000000, 8 * n
    while e:
        if e & 1:
            result = gf_mul(square, result)
        square = gf_mul(square, square)
        e >>= 1
    return result


def _byte_table():
    table = []
    for v in range(256):
        c = v
        for _ in range(8):
            c = (c >> 1) ^ (POLY if c & 1 else 0)
        table.append(c)
    return table


TABLE = _byte_table()


def raw_crc(data, state=0):
    """CRC register after ``data`` from ``state``: no initial value, no final xor."""
    for byte in data:
        state = (state >> 8) ^ TABLE[(state ^ byte) & 0xFF]
    return state


ROW = xpow8n(1024)


def span_partial(span, lane_shift=lambda r, lane: (r - 1 - lane) & 63):
    """The wave's XOR for one span: its raw CRC at the span's end."""
    slots = len(span) // 16
    total = 0
    for lane in range(64):
        acc = 0
        for slot in range(lane, slots, 64):
            acc = gf_mul(ROW, acc) ^ raw_crc(span[16 * slot:16 * slot + 16])
        x = gf_mul(xpow8n(16 * lane_shift(slots & 63, lane)), acc)
        if len(span) & 8:
            x = gf_mul(xpow8n(8), x)
            if lane == 0:
                x ^= raw_crc(span[16 * slots:])
        total ^= x
    return total


def record_crc(record, spans, **kwargs):
    """The finish kernel: every span moved to the record's end, then the initial ~0's term and the final xor."""
    size, s = len(record), 0
    for offset, length in spans:
        s ^= gf_mul(xpow8n(size - offset - length), span_partial(record[offset:offset + length], **kwargs))
    return ~(gf_mul(xpow8n(size), 0xFFFFFFFF) ^ s) & 0xFFFFFFFF


def tiling(lengths):
    spans, offset = [], 0
    for length in lengths:
        spans.append((offset, length))
        offset += length
    return spans, offset


# Span lengths (bytes): one 8-byte word; one slot and a word; 3 slots; 63 slots; one whole row; a row and a
# slot; 80 slots (a short last row of 16); two rows and a word; 4 KiB (4 rows).
LENGTHS = [8, 24, 48, 1008, 1024, 1040, 1280, 2056, 4096]


def test_the_lane_scheme_gives_the_records_crc32c_for_every_span_length_class():
    rng = random.Random(11)
    for lengths in ([n] for n in LENGTHS):
        spans, size = tiling(lengths)
        record = bytes(rng.randrange(256) for _ in range(size))
        assert record_crc(record, spans) == oracle.crc32c(record), lengths
    spans, size = tiling(LENGTHS + LENGTHS[::-1])       # a record of 18 unequal spans
    record = bytes(rng.randrange(256) for _ in range(size))
    assert record_crc(record, spans) == oracle.crc32c(record)


def test_a_whole_rows_lane_shift_fails_on_a_short_last_row():
    rng = random.Random(12)
    spans, size = tiling([1280])                         # 80 slots: r = 16
    record = bytes(rng.randrange(256) for _ in range(size))
    assert record_crc(record, spans, lane_shift=lambda r, lane: 63 - lane) != oracle.crc32c(record)
    spans, size = tiling([1024])                         # whole rows: both shifts agree
    record = bytes(rng.randrange(256) for _ in range(size))
    assert record_crc(record, spans, lane_shift=lambda r, lane: 63 - lane) == oracle.crc32c(record)


def test_the_finish_kernel_s_three_table_shift_equals_shifting_zero_bytes():
    """restore_checked_finish_kernel's x^(8 n) for n < 2^36 is the product of three table entries, x^(8 j),
    x^(8 * 2^12 j) and x^(8 * 2^24 j) with j < 4096, each table built by repeated multiplication from x^0.
    Checked against appending n zero bytes to a register (the definition) for small n, and against squaring for
    large n; a table built one step short (x^(8 (j - 1))) must fail."""
    steps = [xpow8n(1), xpow8n(1 << 12), xpow8n(1 << 24)]
    tables = []
    for step in steps:
        table = [0x80000000]
        for _ in range(4095):
            table.append(gf_mul(table[-1], step))
        tables.append(table)

    def three(n, t=tables):
        return gf_mul(gf_mul(t[0][n & 4095], t[1][(n >> 12) & 4095]), t[2][(n >> 24) & 4095])

    rng = random.Random(41)
    for n in [0, 1, 2, 7, 4095, 4096, 4097, 9000] + [rng.randrange(1 << 14) for _ in range(6)]:
        state = rng.getrandbits(32)
        assert gf_mul(three(n), state) == raw_crc(bytes(n), state), n
    for n in [2359296, 2359296 - 65536, (1 << 36) - 1, rng.randrange(1 << 36)]:
        assert three(n) == xpow8n(n), n
    short = [[t[0]] + t[:-1] for t in tables]
    assert three(9000, short) != three(9000)
