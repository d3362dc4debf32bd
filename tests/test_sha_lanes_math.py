"""The SHA-256 kernel's two-lane scheme, replayed on the CPU against hashlib.

The kernel (kvsnap_amd/csrc/kernels.hip, sha_slot / sha_block_turn /
sha_lanes_start / sha_lanes_finish) splits each record's chain over an
e-lane holding (e, f, g, h) and an a-lane holding (a, b, c, d), the a-half
two rounds behind.  Every slot both lanes run the same formulas on their own
registers X0..X3 with per-lane constants (rotations, the Ch/Maj mask m, and
the word: W[t] + K[t] on the e-lane, 1 on the a-lane) and add the partner's
X1.  Between blocks the e-lane feeds forward first; slots 0 and 1 then finish
the previous block on the a-lane, whose feed-forward follows.  A launch's
first block starts the a-lane from (c, d, y2, y3), chosen so that its slots
0 and 1 produce b and a.

This replays that instruction stream lane by lane (the kernel's own
operations, 32-bit wrapping) over whole messages and over series of block
ranges whose chaining state goes through memory between launches, and checks
every digest against hashlib (FIPS 180-4).  Variants with a plausible mistake
in the scheme (the partner's X0 instead of X1, the missing chaining-word
correction of slots 0 and 1, the feed-forwards in one step) must fail.
"""
import hashlib
import random

import pytest

MASK = 0xFFFFFFFF
K = [
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2,
]
IV = [0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19]


def rotr(x, n):
    return ((x >> n) | (x << (32 - n))) & MASK


def blocks_of(message):
    """FIPS 180-4 padding, then the message schedule W[0..63] + K of each 64-byte block."""
    padded = message + b"\x80" + b"\x00" * ((55 - len(message)) % 64) + (8 * len(message)).to_bytes(8, "big")
    out = []
    for i in range(0, len(padded), 64):
        w = [int.from_bytes(padded[i + 4 * j:i + 4 * j + 4], "big") for j in range(16)]
        for t in range(16, 64):
            s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3)
            s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10)
            w.append((w[t - 16] + s0 + w[t - 7] + s1) & MASK)
        out.append([(w[t] + K[t]) & MASK for t in range(64)])
    return out


class Lane:
    """One lane's registers and constants: X0..X3, the chaining words (E on the e-lane, F on the a-lane)."""

    def __init__(self, a_lane):
        self.a = a_lane
        self.r = (2, 13, 22) if a_lane else (6, 11, 25)
        self.m = MASK if a_lane else 0
        self.x = [0, 0, 0, 0]
        self.chain = [0, 0, 0, 0]

    def sigma(self, x0):
        return rotr(x0, self.r[0]) ^ rotr(x0, self.r[1]) ^ rotr(x0, self.r[2])

    def choose(self, x0, x1, x2):
        u = (~(x0 ^ x1) & MASK) if self.m else x0          # m ? ~(x0 ^ x1) : x0
        return (u & x1) | (~u & MASK & x2)                  # u ? x1 : x2

    def finish(self, w):
        v = (self.sigma(self.x[0]) + self.choose(*self.x[:3]) + w) & MASK
        self.x = [v] + self.x[:3]


class Pair:
    """The e-lane and a-lane of one record, run through the kernel's slots."""

    def __init__(self, h, *, partner_reg=1, correct_turn=True, split_feed_forward=True):
        self.e, self.a = Lane(False), Lane(True)
        self.partner_reg, self.correct_turn, self.split = partner_reg, correct_turn, split_feed_forward
        a, b, c, d, e, f, g, hh = h
        # sha_lanes_start: y2, y3 from the a-lane's constants; the partner's X0 and X1 before any feed-forward.
        y2 = (self.a.sigma(b) + self.a.choose(b, c, d) + e - a) & MASK
        y3 = (self.a.sigma(c) + self.a.choose(c, d, y2) + f - b) & MASK
        self.a.x = [c, d, y2, y3]
        self.e.x = [e, f, g, hh]

    def word_z(self, lane, word):
        return ((lane.x[3] ^ lane.m) + word) & MASK                                    # v_xad_u32

    def slot(self, word_e):
        reg = self.partner_reg
        we = (self.word_z(self.e, word_e) + self.a.x[reg]) & MASK                      # DPP row_half_mirror
        wa = (self.word_z(self.a, 1) + self.e.x[reg]) & MASK
        self.e.finish(we)
        self.a.finish(wa)

    def feed_forward(self, lane):
        lane.x = [(x + c) & MASK for x, c in zip(lane.x, lane.chain)]
        lane.chain = list(lane.x)

    def turn(self, word0, word1):
        unfed0, unfed1 = self.e.x[0], self.e.x[1]
        self.feed_forward(self.e)
        if not self.split:
            self.feed_forward(self.a)
        for word, fw, unfed in ((word0, self.a.chain[3], unfed1), (word1, self.a.chain[2], unfed0)):
            fix = fw if self.correct_turn and self.split else 0
            we = (self.word_z(self.e, word) + ((self.a.x[1] + fix) & MASK)) & MASK     # from_a_partner(x1 + fw)
            wa = (self.word_z(self.a, 1) + unfed) & MASK                               # from_e_partner(unfed)
            self.e.finish(we)
            self.a.finish(wa)
        if self.split:
            self.feed_forward(self.a)

    def block(self, wk):
        self.turn(wk[0], wk[1])
        for t in range(2, 64):
            self.slot(wk[t])

    def end(self):
        """sha_lanes_finish: the chaining value, a-lane words then e-lane words."""
        self.turn(1, 1)
        return self.a.chain + self.e.chain


def digest(message, *, ranges=None, **variant):
    blocks = blocks_of(message)
    ranges = ranges or [(0, len(blocks))]
    h = list(IV)
    for b0, b1 in ranges:                   # one launch per range; the chaining state goes through memory
        pair = Pair(h, **variant)
        for wk in blocks[b0:b1]:
            pair.block(wk)
        h = pair.end()
    return b"".join(v.to_bytes(4, "big") for v in h)


LENGTHS = [0, 1, 3, 55, 56, 63, 64, 65, 119, 120, 128, 200, 1000]


@pytest.mark.parametrize("length", LENGTHS)
def test_the_two_lane_scheme_gives_hashlib_s_digest(length):
    message = random.Random(length).randbytes(length)
    assert digest(message) == hashlib.sha256(message).digest()


def test_ranges_chained_through_memory_give_the_same_digest():
    message = random.Random(7).randbytes(700)            # 11 blocks with the padding
    n = len(blocks_of(message))
    want = hashlib.sha256(message).digest()
    for cuts in ([0, 1, n], [0, 4, 8, n], [0, n - 1, n], [0] + list(range(1, n)) + [n]):
        assert digest(message, ranges=list(zip(cuts, cuts[1:]))) == want, cuts


@pytest.mark.parametrize("variant", [dict(partner_reg=0), dict(correct_turn=False), dict(split_feed_forward=False)],
                         ids=["partner-x0", "no-turn-correction", "feed-forward-together"])
def test_a_scheme_with_a_plausible_mistake_fails(variant):
    message = random.Random(3).randbytes(300)
    assert digest(message, **variant) != hashlib.sha256(message).digest()
