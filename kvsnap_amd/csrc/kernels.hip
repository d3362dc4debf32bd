// gfx950 kernels of the KV snapshot dataplane, behind a plain C ABI.
//
//   restore  packed records (pinned host memory, read in place over the host
//            link, or a device staging buffer) -> each (block, span) written
//            to span_base + block_id * span_pitch.  Replaces the reference's
//            Triton restore kernel (kvsnap/connector/copy_kernel.py:22-49).
//   gather   the inverse: KV cache spans -> block-major packed records.
//            Replaces save_gather's index_select + cat
//            (kvsnap/connector/dataplane.py:409-417).
//   zero     byte ranges of a record set to zero: the token slots past the last
//            computed token (kvsnap/connector/dataplane.py:262-272).
//   crc32c   per-record CRC32C (reflected 0x82F63B78, init/xorout ~0), bit
//            exact with csrc/dataplane/io.cpp:16-47.
//   sha256   per-record SHA-256 digest, the blob id of
//            kvsnap/connector/volatile.py:151 and kvsnap/store/store.py:622.
//   synth    seeded synthetic KV bytes (bench and test input only).
//
// A "span" is one contiguous run of a block inside one cache tensor: one per
// layer for [blocks, H, N, C] caches (the reference's layout), two per layer
// (K then V) for [2, blocks, N, H, C] caches.  Span s of block b lives at
// span_base[s] + b * span_pitch[s], is span_words[s] 8-byte words long and
// sits at byte span_offset[s] of the block's packed record.  All tables are
// int64 arrays in device memory, as in the reference's launch contract.
//
// No MFMA anywhere: nothing on this path is a contraction.  The copies are
// 16-byte-per-lane streams (4 or 8 dwordx4 loads in flight per lane), the CRC
// is LDS table lookups combined in GF(2), and SHA-256 runs one record per two
// lanes because the hash is a sequential chain within a record.
#include <hip/hip_runtime.h>

#include "common.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;   // CRC, zero and synthetic-fill workgroups: 4 waves

// ----------------------------------------------------------------- copies

// Copy nbytes (a multiple of 8; src and dst 8-byte aligned) with `lanes`
// lanes of the workgroup (this one is `lane`), kU dwordx4 loads in flight per
// lane.  The 16-byte path covers everything when both ends are 16-byte
// aligned, which the host tables normally guarantee; an 8-byte tail covers
// the rest.
template <int kU>
__device__ __forceinline__ void copy_span(const char* __restrict__ src, char* __restrict__ dst, int64_t nbytes,
                                          int lane, int lanes) {
    int64_t done = 0;
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
        const u32x4* s = reinterpret_cast<const u32x4*>(src);
        u32x4* d = reinterpret_cast<u32x4*>(dst);
        const int64_t nv = nbytes >> 4;
        int64_t i = lane;
        for (; i + (kU - 1) * lanes < nv; i += kU * lanes) {
            u32x4 v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) v[u] = __builtin_nontemporal_load(s + i + u * lanes);
#pragma unroll
            for (int u = 0; u < kU; ++u) __builtin_nontemporal_store(v[u], d + i + u * lanes);
        }
        // Fewer than kU vectors left for this lane: still every load before any store.
        if (i < nv) {
            u32x4 v[kU] = {};
#pragma unroll
            for (int u = 0; u < kU; ++u)
                if (i + u * lanes < nv) v[u] = __builtin_nontemporal_load(s + i + u * lanes);
#pragma unroll
            for (int u = 0; u < kU; ++u)
                if (i + u * lanes < nv) __builtin_nontemporal_store(v[u], d + i + u * lanes);
        }
        done = nv << 4;
    }
    const uint64_t* s8 = reinterpret_cast<const uint64_t*>(src + done);
    uint64_t* d8 = reinterpret_cast<uint64_t*>(dst + done);
    const int64_t nw = (nbytes - done) >> 3;
    for (int64_t i = lane; i < nw; i += lanes) d8[i] = s8[i];
}

// Jobs are (block, span) pairs, job j = (block j / n_spans, span j % n_spans):
// the reference kernel's order (copy_kernel.py:29-31), so a launch walks its
// records front to back.  A workgroup copies kT >> lane_shift jobs at a time,
// one per group of 2^lane_shift lanes.  The host picks lane_shift from the
// shortest span: the whole workgroup for the 32-64 KiB spans of a full bf16
// cache, down to one wave for the 4 KiB spans of a tensor-parallel shard, so
// that a pass keeps about kT * kU loads in flight whatever the span length.
// A group is at least one wave, so its job index (and the table reads that
// follow from it) is wave-uniform.
struct JobLanes {
    int lane, lanes, group, per_pass;
};

template <int kT>
__device__ __forceinline__ JobLanes job_lanes(int lane_shift) {
    JobLanes j;
    j.lanes = 1 << lane_shift;
    j.per_pass = kT >> lane_shift;
    j.group = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> lane_shift);
    j.lane = static_cast<int>(threadIdx.x) & (j.lanes - 1);
    return j;
}

// Restore: reads cross the host link, so a small persistent grid of 256-lane
// workgroups with 8 loads in flight per lane keeps it full while leaving the
// CUs to the engine.
constexpr int kRestoreThreads = 256, kRestoreUnroll = 8;
// Gather with a fixed grid or an unknown span length (the pieces kernel below
// takes the rest): HBM to HBM, 1024-lane workgroups with 4 loads in flight
// per lane (64 KiB per pass), the fastest shape of this kind measured.  A
// 32 KiB span takes the whole workgroup, 2 loads per lane.  Tried and slower
// on the 8k Qwen3-8B gather: an unroll of 8 (512 lanes per span, 4 loads
// each; 106 SGPRs, one workgroup per CU: 5.1 against 5.9 TB/s), and
// global-address-space loads and stores in place of the flat ones the table
// addresses compile to (equal on 32 KiB spans, 5.6 against 5.9 TB/s on 64 KiB
// ones).
constexpr int kGatherThreads = 1024, kGatherUnroll = 4;
// Scatter from device records: HBM to HBM like the gather, writes scattered.
constexpr int kScatterThreads = 1024, kScatterUnroll = 4;

__global__ __launch_bounds__(kRestoreThreads) void restore_kernel(
    const int64_t* __restrict__ sources, const int64_t* __restrict__ blocks, int64_t n_blocks,
    const int64_t* __restrict__ offs, const int64_t* __restrict__ bases, const int64_t* __restrict__ pitches,
    const int64_t* __restrict__ words, int64_t n_spans, int lane_shift) {
    const JobLanes jl = job_lanes<kRestoreThreads>(lane_shift);
    const int64_t jobs = n_blocks * n_spans;
    for (int64_t job = static_cast<int64_t>(blockIdx.x) * jl.per_pass + jl.group; job < jobs;
         job += static_cast<int64_t>(gridDim.x) * jl.per_pass) {
        const int64_t b = job / n_spans, s = job - b * n_spans;
        const char* src = reinterpret_cast<const char*>(sources[b] + offs[s]);
        char* dst = reinterpret_cast<char*>(bases[s] + blocks[b] * pitches[s]);
        copy_span<kRestoreUnroll>(src, dst, words[s] * 8, jl.lane, jl.lanes);
    }
}

__global__ __launch_bounds__(kGatherThreads) void gather_kernel(
    const int64_t* __restrict__ blocks, int64_t n_blocks, const int64_t* __restrict__ offs,
    const int64_t* __restrict__ bases, const int64_t* __restrict__ pitches, const int64_t* __restrict__ words,
    int64_t n_spans, char* __restrict__ records, int64_t record_pitch, int lane_shift) {
    const JobLanes jl = job_lanes<kGatherThreads>(lane_shift);
    const int64_t jobs = n_blocks * n_spans;
    for (int64_t job = static_cast<int64_t>(blockIdx.x) * jl.per_pass + jl.group; job < jobs;
         job += static_cast<int64_t>(gridDim.x) * jl.per_pass) {
        const int64_t b = job / n_spans, s = job - b * n_spans;
        const char* src = reinterpret_cast<const char*>(bases[s] + blocks[b] * pitches[s]);
        char* dst = records + b * record_pitch + offs[s];
        copy_span<kGatherUnroll>(src, dst, words[s] * 8, jl.lane, jl.lanes);
    }
}

// Scatter from packed records in device memory (HBM to HBM, the verified
// restore's last step): the gather's inverse, with its shape.  Workgroups are
// dealt to the 8 XCDs round robin (workgroup i runs on XCD i % 8); here each
// XCD takes one contiguous range of passes, so a record's spans are read
// through one XCD's L2.  That measured 5.66 TB/s against 5.26 with the passes
// dealt round robin; the gather, whose writes are the contiguous side, gained
// nothing.
constexpr int kXcds = 8;

__global__ __launch_bounds__(kScatterThreads) void scatter_kernel(
    const char* __restrict__ records, int64_t record_pitch, const int64_t* __restrict__ blocks, int64_t n_blocks,
    const int64_t* __restrict__ offs, const int64_t* __restrict__ bases, const int64_t* __restrict__ pitches,
    const int64_t* __restrict__ words, int64_t n_spans, int lane_shift) {
    const JobLanes jl = job_lanes<kScatterThreads>(lane_shift);
    const int64_t jobs = n_blocks * n_spans;
    const int64_t passes = (jobs + jl.per_pass - 1) / jl.per_pass;
    const int64_t grid = gridDim.x;
    int64_t first = blockIdx.x, end = passes, stride = grid;
    if (grid >= kXcds) {
        const int64_t per_xcd = (passes + kXcds - 1) / kXcds;
        const int64_t xcd = blockIdx.x % kXcds;
        first = xcd * per_xcd + blockIdx.x / kXcds;
        end = (xcd + 1) * per_xcd < passes ? (xcd + 1) * per_xcd : passes;
        stride = (grid - xcd + kXcds - 1) / kXcds;  // workgroups on this XCD
    }
    for (int64_t pass = first; pass < end; pass += stride) {
        const int64_t job = pass * jl.per_pass + jl.group;
        if (job >= jobs) continue;  // only in the last pass
        const int64_t b = job / n_spans, s = job - b * n_spans;
        const char* src = records + b * record_pitch + offs[s];
        char* dst = reinterpret_cast<char*>(bases[s] + blocks[b] * pitches[s]);
        copy_span<kScatterUnroll>(src, dst, words[s] * 8, jl.lane, jl.lanes);
    }
}

// Gather and scatter in pieces: one wave per KiB of a span, one 16-byte load
// and one store per lane.  Workgroup (x, b) copies piece x % pieces of span
// x / pieces of block b (dispatched x first, so in the jobs' order above).  A
// span's last piece takes every byte from its KiB to the span's end, so
// `pieces` (the host's ceil(shortest span / 1 KiB)) shapes the launch without
// changing what is copied: a longer span's last wave loops over the rest,
// and a piece past a span's end copies nothing.  On the 8k Qwen3-8B gather (36,864 spans of 32 KiB) this shape ran
// at 6.5 TB/s, against 5.7-5.8 for one 1024-lane workgroup per span
// (gather_kernel above) and 6.2 for 256-lane workgroups per 4 KiB piece.
// Each wave lives for one load and one store, and the dispatcher keeps the
// CUs full of them.  Pieces dealt to the XCDs in contiguous ranges ran at
// 6.35 TB/s, so consecutive pieces go round robin.
constexpr int kPieceBytes = 64 * 16;

template <bool kGather>
__device__ __forceinline__ void copy_piece(const int64_t* __restrict__ blocks, const int64_t* __restrict__ offs,
                                           const int64_t* __restrict__ bases, const int64_t* __restrict__ pitches,
                                           const int64_t* __restrict__ words, uint32_t pieces,
                                           char* __restrict__ records, int64_t record_pitch) {
    const uint32_t b = blockIdx.y, s = blockIdx.x / pieces, p = blockIdx.x - s * pieces;
    const int64_t length = words[s] * 8, at = static_cast<int64_t>(p) * kPieceBytes;
    if (at >= length) return;
    const int64_t end = p + 1 == pieces || length - at < kPieceBytes ? length : at + kPieceBytes;
    char* cache = reinterpret_cast<char*>(bases[s] + blocks[b] * pitches[s]) + at;
    char* record = records + static_cast<int64_t>(b) * record_pitch + offs[s] + at;
    const char* src = kGather ? cache : record;
    char* dst = kGather ? record : cache;
    const int lane = static_cast<int>(threadIdx.x);
    if (end - at == kPieceBytes && ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0)
        __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + lane),
                                    reinterpret_cast<u32x4*>(dst) + lane);
    else
        copy_span<1>(src, dst, end - at, lane, 64);
}

__global__ __launch_bounds__(64) void gather_pieces_kernel(const int64_t* __restrict__ blocks,
                                                           const int64_t* __restrict__ offs,
                                                           const int64_t* __restrict__ bases,
                                                           const int64_t* __restrict__ pitches,
                                                           const int64_t* __restrict__ words, uint32_t pieces,
                                                           char* __restrict__ records, int64_t record_pitch) {
    copy_piece<true>(blocks, offs, bases, pitches, words, pieces, records, record_pitch);
}

__global__ __launch_bounds__(64) void scatter_pieces_kernel(const int64_t* __restrict__ blocks,
                                                            const int64_t* __restrict__ offs,
                                                            const int64_t* __restrict__ bases,
                                                            const int64_t* __restrict__ pitches,
                                                            const int64_t* __restrict__ words, uint32_t pieces,
                                                            char* __restrict__ records, int64_t record_pitch) {
    copy_piece<false>(blocks, offs, bases, pitches, words, pieces, records, record_pitch);
}

// Gather into per-block destinations (pinned host records written in place
// over the host link, or anywhere else): the restore kernel's inverse, with
// its small-grid shape.
__global__ __launch_bounds__(kRestoreThreads) void gather_to_kernel(
    const int64_t* __restrict__ dests, const int64_t* __restrict__ blocks, int64_t n_blocks,
    const int64_t* __restrict__ offs, const int64_t* __restrict__ bases, const int64_t* __restrict__ pitches,
    const int64_t* __restrict__ words, int64_t n_spans, int lane_shift) {
    const JobLanes jl = job_lanes<kRestoreThreads>(lane_shift);
    const int64_t jobs = n_blocks * n_spans;
    for (int64_t job = static_cast<int64_t>(blockIdx.x) * jl.per_pass + jl.group; job < jobs;
         job += static_cast<int64_t>(gridDim.x) * jl.per_pass) {
        const int64_t b = job / n_spans, s = job - b * n_spans;
        const char* src = reinterpret_cast<const char*>(bases[s] + blocks[b] * pitches[s]);
        char* dst = reinterpret_cast<char*>(dests[b] + offs[s]);
        copy_span<kRestoreUnroll>(src, dst, words[s] * 8, jl.lane, jl.lanes);
    }
}

// One wave that sleeps for `iters` rounds of s_sleep 127 (about 3.4 us each
// at 2.4 GHz) and then ends: a fixed count, so every launch finishes.  The
// data plane holds a stream with it for a few milliseconds to see which other
// streams' work waits behind it, i.e. which streams share its hardware queue.
__global__ __launch_bounds__(64) void hold_kernel(int iters) {
    for (int i = 0; i < iters; ++i) __builtin_amdgcn_s_sleep(127);
}

// One workgroup per region; regions are small (one token's C elements).
__global__ __launch_bounds__(kThreads) void zero_kernel(char* __restrict__ base, const int64_t* __restrict__ offsets,
                                                       const int64_t* __restrict__ lengths, int64_t n) {
    for (int64_t r = blockIdx.x; r < n; r += gridDim.x) {
        char* p = base + offsets[r];
        const int64_t len = lengths[r];
        for (int64_t i = threadIdx.x; i < len; i += kThreads) p[i] = 0;
    }
}

// ----------------------------------------------------------------- synthetic KV
// Integer-only generator, bit-identical to the oracle's C version.

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t span_key(uint64_t seed, uint64_t span, uint64_t block) {
    uint64_t h = mix64(seed + 0x9E3779B97F4A7C15ull);
    h = mix64(h + span * 0xD1B54A32D192ED03ull);
    return mix64(h + block * 0xABC98388FB8FAC03ull);
}

__device__ __forceinline__ float normal_sample(uint64_t key, uint64_t element) {
    const uint64_t r = mix64(key + element * 0x9E3779B97F4A7C15ull);
    const int32_t sum = static_cast<int32_t>(r & 0xFFFF) + static_cast<int32_t>((r >> 16) & 0xFFFF) +
                        static_cast<int32_t>((r >> 32) & 0xFFFF) + static_cast<int32_t>(r >> 48);
    return __fmul_rn(static_cast<float>(sum - 131070), 2.6429e-05f);
}

__device__ __forceinline__ uint32_t to_bf16(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t to_e4m3(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x43E00000u) return sign | 0x7Eu;
    if (a < 0x3C800000u) {
        const float q = __fmul_rn(__uint_as_float(a), 512.0f);
        uint32_t n = static_cast<uint32_t>(q);
        const float frac = __fsub_rn(q, static_cast<float>(n));
        if (frac > 0.5f || (frac == 0.5f && (n & 1u))) ++n;
        return sign | n;
    }
    const uint32_t rounded = a + 0x7FFFFu + ((a >> 20) & 1u);
    const uint32_t exp = (rounded >> 23) - 127 + 7;
    const uint32_t man = (rounded >> 20) & 7u;
    uint32_t code = (exp << 3) | man;
    if (code > 0x7Eu) code = 0x7Eu;
    return sign | code;
}

__global__ __launch_bounds__(kThreads) void synth_kernel(uint64_t seed, int kind, const int64_t* __restrict__ bases,
                                                        const int64_t* __restrict__ pitches,
                                                        const int64_t* __restrict__ words,
                                                        const float* __restrict__ inv_scales, int64_t n_spans,
                                                        int64_t first_block, int64_t n_blocks) {
    const int64_t jobs = n_blocks * n_spans;
    for (int64_t job = blockIdx.x; job < jobs; job += gridDim.x) {
        const int64_t b = first_block + job / n_spans, s = job % n_spans;
        u32x4* dst = reinterpret_cast<u32x4*>(bases[s] + b * pitches[s]);
        const int64_t nv = words[s] / 2;  // 16-byte vectors
        const uint64_t key = span_key(seed, static_cast<uint64_t>(s), static_cast<uint64_t>(b));
        const float inv = inv_scales ? inv_scales[s] : 1.0f;
        for (int64_t v = threadIdx.x; v < nv; v += kThreads) {
            uint32_t w[4];
            if (kind == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint64_t e = static_cast<uint64_t>(v) * 8 + 2 * i;
                    w[i] = to_bf16(normal_sample(key, e)) | (to_bf16(normal_sample(key, e + 1)) << 16);
                }
            } else if (kind == 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t word = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint64_t e = static_cast<uint64_t>(v) * 16 + 4 * i + j;
                        word |= to_e4m3(__fmul_rn(normal_sample(key, e), inv)) << (8 * j);
                    }
                    w[i] = word;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint64_t r = mix64(key + (static_cast<uint64_t>(v) * 2 + i) * 0x9E3779B97F4A7C15ull);
                    w[2 * i] = static_cast<uint32_t>(r);
                    w[2 * i + 1] = static_cast<uint32_t>(r >> 32);
                }
            }
            dst[v] = u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

// A stand-in for decode attention's KV traffic: every (sequence, span) job
// streams the span of each block in the sequence's block table (16-byte
// loads) and folds it into a 32-bit sum, one word per job.
__global__ __launch_bounds__(kThreads) void synth_decode_kernel(const int64_t* __restrict__ bases,
                                                               const int64_t* __restrict__ pitches,
                                                               const int64_t* __restrict__ words, int64_t n_spans,
                                                               const int64_t* __restrict__ table, int64_t n_seqs,
                                                               int64_t blocks_per_seq, uint32_t* __restrict__ out) {
    __shared__ uint32_t red[kThreads / 64];
    const int64_t jobs = n_seqs * n_spans;
    for (int64_t job = blockIdx.x; job < jobs; job += gridDim.x) {
        const int64_t q = job / n_spans, s = job - q * n_spans;
        const int64_t nv = words[s] / 2;
        uint32_t acc = 0;
        for (int64_t k = 0; k < blocks_per_seq; ++k) {
            const u32x4* src = reinterpret_cast<const u32x4*>(bases[s] + table[q * blocks_per_seq + k] * pitches[s]);
            for (int64_t v = threadIdx.x; v < nv; v += kThreads) {
                const u32x4 x = src[v];
                acc += x.x ^ x.y ^ x.z ^ x.w;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
        __syncthreads();
        if (threadIdx.x == 0) out[job] = red[0] + red[1] + red[2] + red[3];
        __syncthreads();
    }
}

// ----------------------------------------------------------------- CRC32C
//
// Linear algebra of the reflected CRC (all arithmetic in GF(2)):
//   the register after a message M of N bytes from start value s0 is
//     shift(s0, N) ^ R(M),
//   where shift(s, n) advances s by n zero bytes (multiplication by x^(8n)
//   mod P) and R is the "raw" CRC from a zero register, which is linear and
//   satisfies R(A || B) = shift(R(A), |B|) ^ R(B) and R(0^k || A) = R(A).
// So a record can be cut into equal stripes (the first one padded in front
// with virtual zero bytes) whose raw CRCs are computed independently and
// combined; crc32c = ~(shift(~prior, N) ^ R(record)).
//
// A stripe is one wave's job: `groups` groups of 1 KiB, lane l folding the
// 16-byte word at l * 16 of every group (one coalesced 16-byte load per lane
// and group).  A lane keeps 6 chains, chain c taking the stripe's groups c,
// c + 6, ... (6 loads of a batch in flight, 6 independent lookup streams),
// so a chain's words are 6 KiB apart:
//   acc' = advance(acc) ^ R(word),   advance(s) = shift(s, 6144),
// R(word) the word's raw CRC from a zero register: four slicing-by-4 steps
// that do not wait for acc, so the advance's lookups go out beside theirs.
// At the end the chains are combined by Horner's rule in the order of their
// last groups (shift by one group between them), each lane's register is
// shifted past the lanes after it (per-lane constants), and the wave's XOR is
// the stripe's raw CRC.  The stripes of a record are shifted to its end (in
// the workgroup, or by a combine kernel) and the initial value's term added.
//
//   S[i][v]  = shift(v, 4 - i)                 (slicing-by-4, one dword)
//   Gn[i][v] = shift(v << 4i, 6144)            (the advance, by nibbles)
//   H[k][v]  = shift(v << 8k, 1024)            (the chain behind, one group on)
//   M[l]     = x^(8 * 16 * (63 - l)) mod P     (lane l's word to the group's end)
//
// The lookups are the kernel's cost, and random indices into one shared
// table put several lanes of a wave on one LDS bank.  So every lane reads its
// own copy of S and of Gn, laid out so that lane t's entries all sit in bank
// t % 32 and the 32 lanes an LDS pass serves never share a bank:
//   Gn[i][v] for lane t at byte 4096 + (i / 2) * 4096 + v * 256 + (i % 2) * 128 + (t % 32) * 4,
//   S[i][v]  for lane t at byte 20480 + (i / 2) * 65536 + v * 256 + (i % 2) * 128 + (t % 32) * 4,
// after the shared H at byte 0 (every table's base then fits the 16-bit offset field of ds_read).
// An address is one byte move: v_perm_b32 puts the index (a byte of the
// state, or of its nibbles spread one per byte) into byte 1 of a per-lane
// constant holding the lane's column; the page rides in the instruction's
// offset field.  The advance by nibbles takes 8 lookups where bytes would
// take 4, but 16 tables of 16 entries fit 32 private copies in 16 KiB, where
// the byte tables' copies would need 128 KiB more than the LDS has; shared,
// their conflicts had been 29 % of the LDS's active cycles.  H and the S and
// Gn copies fill 148 KiB of the LDS, so a CU holds one 1024-lane workgroup,
// as many waves as 128 registers a lane allow anyway.
constexpr uint32_t kPoly = 0x82F63B78u;
constexpr int kCrcThreads = 1024;
constexpr int kCrcWaves = kCrcThreads / 64;
constexpr int kCrcRun = 16;                  // bytes one lane folds per group: one 16-byte word
constexpr int kCrcChains = 6;                // groups per batch, each its own chain
constexpr int kCrcLoadPolicy = 2;           // the buffer loads' cache-policy bits: nt, streaming loads
constexpr int kCrcRunWords = kCrcRun / 16;
constexpr int kCrcBatchWords = kCrcChains * kCrcRunWords;  // 16-byte loads per lane per batch
constexpr int kCrcGroup = 64 * kCrcRun;      // one wave's group
constexpr int kCrcMaxStripes = 64;           // per record: the combine's lanes
constexpr int kCrcResidentWaves = 256 * kCrcWaves;  // one workgroup per CU
constexpr int kCrcBehindBytes = 4 * 1024;    // H, shared, at LDS byte 0
constexpr int kCrcAdvanceBytes = 16 * 1024;  // the lanes' copies of Gn, after H
constexpr int kCrcPrivateBytes = 2 * 65536;  // the lanes' copies of S, after Gn
constexpr int kCrcGnAt = kCrcBehindBytes / 4;                        // in words
constexpr int kCrcSAt = (kCrcBehindBytes + kCrcAdvanceBytes) / 4;    // in words

// g_crc_tables: S[4][256], then Gn[8][16], then H[4][256], then M[64].
constexpr int kCrcAdvance = 4 * 256;
constexpr int kCrcBehind = kCrcAdvance + 8 * 16;
constexpr int kCrcLaneShift = kCrcBehind + 4 * 256;
constexpr int kCrcTableWords = kCrcLaneShift + 64;

__device__ uint32_t g_crc_tables[kCrcTableWords];

__device__ __forceinline__ uint32_t gf_mul(uint32_t a, uint32_t b) {
    // a * b mod P in the reflected representation (bit 31 is x^0).
    uint32_t p = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        p ^= b & (0u - ((a >> (31 - i)) & 1u));
        b = (b >> 1) ^ (kPoly & (0u - (b & 1u)));
    }
    return p;
}

__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ uint32_t lds_word(const uint32_t* lds, uint32_t byte) {
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(lds) + byte);
}

// The per-lane address constant: byte 0 = the lane's column in S[0], S[2] and
// the even Gn tables, byte 1 = its column in S[1], S[3] and the odd Gn tables,
// byte 2 = 1 (S's second 64 KiB).
__device__ __forceinline__ uint32_t crc_columns(uint32_t lane) {
    const uint32_t col = (lane & 31u) * 4u;
    return col | ((col + 128u) << 8) | (1u << 16);
}

// shift(acc, d) for the distance d of the shared byte tables at `lds` (H).
__device__ __forceinline__ uint32_t crc_advance(const uint32_t* lds, uint32_t acc) {
    return xor3(lds_word(lds, (acc & 0xFFu) << 2), lds_word(lds, 1024u + (((acc >> 8) & 0xFFu) << 2)),
                lds_word(lds, 2048u + (((acc >> 16) & 0xFFu) << 2))) ^
           lds_word(lds, 3072u + ((acc >> 24) << 2));
}

// The run of lane `lane` in the group at record offset `group_at` (which may
// lie partly or wholly in the front padding: those bytes are zero).
template <bool kAligned>
__device__ __forceinline__ void crc_load_run(const uint8_t* __restrict__ rec, int64_t group_at, uint32_t lane,
                                             u32x4* v) {
    const int64_t at = group_at + static_cast<int64_t>(lane) * kCrcRun;
#pragma unroll
    for (int k = 0; k < kCrcRunWords; ++k) {
        v[k] = u32x4{0u, 0u, 0u, 0u};
        const int64_t word = at + 16 * k;
        if (kAligned) {
            // The padding is a multiple of 16 here, so a word is all padding or all record.
            if (word >= 0) v[k] = *reinterpret_cast<const u32x4*>(rec + word);
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
            for (int b = 0; b < 16; ++b)
                if (word + b >= 0) w[b >> 2] |= static_cast<uint32_t>(rec[word + b]) << (8 * (b & 3));
            v[k] = u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

// Global-address-space views of memory, for record addresses the kernels pass through an empty asm
// statement (crc_opaque): loads through a kernel argument's pointer count as invariant, and the compiler
// moved them past the table fill and its barrier, to where they are used.
using GlobalByte = const __attribute__((address_space(1))) uint8_t;
using GlobalWord = const __attribute__((address_space(1))) u32x4;

__device__ __forceinline__ GlobalByte* crc_opaque(const void* p) {
    GlobalByte* g = (GlobalByte*)p;
    asm volatile("" : "+s"(g));
    return g;
}

// A wave-uniform 64-bit value moved to scalar registers (lane 0's copy).
__device__ __forceinline__ uint64_t uniform64(uint64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// A raw buffer resource over [base, base + bytes) (stride 0, so a load past `bytes` reads zeros).
// kBufferWord3 is the descriptor's last dword on gfx9: data format 32 in bits 15-18, every other field zero.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t crc_buffer(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferWord3);
}

// A batch of whole groups of record bytes at record offset `at` (>= 0): chain c's run at v[c].  Buffer
// loads: the record's address and the batch's offset in scalar registers, each lane's offset (lane * 16,
// the same every batch) in one vector register.  With a 64-bit address per lane in vector registers the
// compiler put an `s_waitcnt vmcnt(0)` at the head of the batch loop, before the next batch was issued, so
// the loads in flight drained every other batch.  The resource ends at the batch's end: a load past it
// would read zeros, never another allocation.
__device__ __forceinline__ void crc_load_batch(const uint8_t* __restrict__ rec, int64_t at, uint32_t lane, u32x4* v) {
    static_assert(kCrcRunWords == 1, "one word per chain and batch");
    const __amdgpu_buffer_rsrc_t buffer =
        crc_buffer(rec + at, static_cast<uint32_t>(kCrcChains * kCrcGroup));
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c)
        v[c] = __builtin_amdgcn_raw_buffer_load_b128(buffer, lane * kCrcRun, c * kCrcGroup, kCrcLoadPolicy);
}

// Any batch: the first may hold front padding, the last may hold fewer than kCrcChains groups.
template <bool kAligned>
__device__ __forceinline__ void crc_load_any(const uint8_t* __restrict__ rec, int64_t at, int count, uint32_t lane,
                                             u32x4* v) {
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c) {
        if (c < count) {
            crc_load_run<kAligned>(rec, at + static_cast<int64_t>(c) * kCrcGroup, lane, v + c * kCrcRunWords);
        } else {
#pragma unroll
            for (int k = 0; k < kCrcRunWords; ++k) v[c * kCrcRunWords + k] = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

// One dword through slicing-by-4 looks up the four bytes of x = state ^
// dword.  v_perm_b32 picks bytes of {S0 = x (bytes 4-7), S1 = cols (bytes
// 0-3)}, selector 12 giving 0x00: the address of S[i][byte i of x] is byte i
// of x in byte 1 above the lane's column, one instruction per lookup:
//   S[0]: ((x & 0xFF) << 8) | col                    selector 0x0C0C0400
//   S[1]: (x & 0xFF00) | (col + 128)                  selector 0x0C0C0501
//   S[2]: 0x10000 | ((x >> 8) & 0xFF00) | col          selector 0x0C020600
//   S[3]: 0x10000 | ((x >> 16) & 0xFF00) | (col + 128) selector 0x0C020701
// Every chain's lookups of a step are issued before any result is used, so
// a wave keeps 4 * kCrcChains LDS reads in flight (left to itself the
// compiler runs the chains one after another, each step waiting out a whole
// LDS round trip).

// The advance of one chain, issued: Gn's eight lookups of `x` (nibble 2k is byte k of `lo`, nibble 2k + 1
// byte k of `hi`; Gn[2k] and Gn[2k + 1] share page k, columns col and col + 128: bytes 0 and 1 of `cols`).
__device__ __forceinline__ void crc_advance_issue(const uint32_t* lds, uint32_t cols, uint32_t x, uint32_t* r) {
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    const uint32_t* gn = lds + kCrcGnAt;
    r[0] = lds_word(gn, __builtin_amdgcn_perm(lo, cols, 0x0C0C0400u));
    r[1] = lds_word(gn, __builtin_amdgcn_perm(hi, cols, 0x0C0C0401u));
    r[2] = lds_word(gn + 1024, __builtin_amdgcn_perm(lo, cols, 0x0C0C0500u));
    r[3] = lds_word(gn + 1024, __builtin_amdgcn_perm(hi, cols, 0x0C0C0501u));
    r[4] = lds_word(gn + 2048, __builtin_amdgcn_perm(lo, cols, 0x0C0C0600u));
    r[5] = lds_word(gn + 2048, __builtin_amdgcn_perm(hi, cols, 0x0C0C0601u));
    r[6] = lds_word(gn + 3072, __builtin_amdgcn_perm(lo, cols, 0x0C0C0700u));
    r[7] = lds_word(gn + 3072, __builtin_amdgcn_perm(hi, cols, 0x0C0C0701u));
}

// Fold a batch: chain c takes word v[c], acc' = shift(acc, kCrcChains KiB) ^ R(word), R the word's raw
// CRC from a zero register in four slicing-by-4 steps.  R does not depend on acc, so the advances' lookups (a
// quarter of the chains beside each step) ride along with the steps': four LDS round trips per batch, where
// advancing first and then stepping from the advanced register takes five.  Chains past `count` (the
// last batch's missing groups) are left alone.
__device__ __forceinline__ void crc_fold_batch(const uint32_t* lds, uint32_t cols, const u32x4* v, uint32_t* acc,
                                               int count) {
    static_assert(kCrcRunWords == 1, "one word per chain and batch");
    constexpr int kQuarter = (kCrcChains + 3) / 4;
    const uint32_t* tab = lds + kCrcSAt;
    uint32_t t[kCrcChains], g[kCrcChains];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t r[kCrcChains][4], q[kQuarter][8];
#pragma unroll
        for (int c = 0; c < kCrcChains; ++c) {
            const uint32_t d = k == 0 ? v[c].x : k == 1 ? v[c].y : k == 2 ? v[c].z : v[c].w;
            const uint32_t x = k == 0 ? d : t[c] ^ d;
            r[c][0] = lds_word(tab, __builtin_amdgcn_perm(x, cols, 0x0C0C0400u));
            r[c][1] = lds_word(tab, __builtin_amdgcn_perm(x, cols, 0x0C0C0501u));
            r[c][2] = lds_word(tab, __builtin_amdgcn_perm(x, cols, 0x0C020600u));
            r[c][3] = lds_word(tab, __builtin_amdgcn_perm(x, cols, 0x0C020701u));
        }
#pragma unroll
        for (int i = 0; i < kQuarter; ++i)
            if (k * kQuarter + i < kCrcChains) crc_advance_issue(lds, cols, acc[k * kQuarter + i], q[i]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < kCrcChains; ++c) t[c] = xor3(r[c][0], r[c][1], r[c][2]) ^ r[c][3];
#pragma unroll
        for (int i = 0; i < kQuarter; ++i)
            if (k * kQuarter + i < kCrcChains)
                g[k * kQuarter + i] =
                    xor3(xor3(q[i][0], q[i][1], q[i][2]), xor3(q[i][3], q[i][4], q[i][5]), q[i][6]) ^ q[i][7];
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c)
        if (c < count) acc[c] = g[c] ^ t[c];
}

// The batches of one stripe after its first (already in `cur`, `count` groups, folded next), with the
// batch after the current one loaded while the current one is folded (two register buffers).  In the
// steady state every prefetch is a whole batch of record bytes and unconditional, so the wait for the
// current batch lets the prefetch's loads stay in flight.  The last batch may hold fewer groups than
// chains; it is loaded once the one before it is folded.
template <bool kAligned>
__device__ __forceinline__ void crc_fold_rest(const uint32_t* lds, uint32_t cols, const uint8_t* __restrict__ rec,
                                              int64_t start, int groups, int g, int count, uint32_t lane, u32x4* cur,
                                              uint32_t* acc) {
    crc_fold_batch(lds, cols, cur, acc, count);
    g += kCrcChains;
    if (g < groups) {
        const int left = groups - g;
        crc_load_any<kAligned>(rec, start + static_cast<int64_t>(g) * kCrcGroup, left, lane, cur);
        crc_fold_batch(lds, cols, cur, acc, left);
    }
}

// The LDS tables of a CRC workgroup: H shared at byte 0, then the lanes'
// private copies of Gn and of S.  S entry (table, v) is a 128-byte run (its
// 32 lane columns) at (table / 2) * 64 KiB + v * 256 + (table % 2) * 128.
// The fill writes S as 16-byte chunks in address order, chunk k * 1024 + t
// from thread t, so the 64 lanes of each write cover 1 KiB of consecutive
// banks; one lane per entry (its run's eight chunks) put a wave's lanes 256
// bytes apart, all on the same four banks, and took about 4 us a launch.
// Gn is written eight threads per entry (128 consecutive bytes), H one word
// per thread.
constexpr int kCrcFillChunks = kCrcPrivateBytes / 16 / kCrcThreads;  // S chunks per thread

struct CrcTableWords {
    uint32_t s[kCrcFillChunks], advance, behind;
};

__device__ __forceinline__ uint32_t crc_fill_entry(uint32_t chunk) {
    const uint32_t half = chunk >> 12, r = chunk & 4095u;
    return (2u * half + ((r >> 3) & 1u)) * 256u + (r >> 4);  // table * 256 + v
}

__device__ __forceinline__ CrcTableWords crc_table_words() {
    static_assert(kCrcThreads == 4 * 256, "one thread per H entry");
    static_assert(kCrcFillChunks * kCrcThreads * 16 == kCrcPrivateBytes, "S chunks split evenly");
    const uint32_t t = threadIdx.x;
    CrcTableWords w;
#pragma unroll
    for (int k = 0; k < kCrcFillChunks; ++k) w.s[k] = g_crc_tables[crc_fill_entry(k * kCrcThreads + t)];
    w.advance = g_crc_tables[kCrcAdvance + (t >> 3)];
    w.behind = g_crc_tables[kCrcBehind + t];
    return w;
}

__device__ __forceinline__ void crc_fill_tables(uint32_t* lds, const CrcTableWords& w) {
    const uint32_t t = threadIdx.x;
    u32x4* chunks = reinterpret_cast<u32x4*>(lds + kCrcSAt);
#pragma unroll
    for (int k = 0; k < kCrcFillChunks; ++k) chunks[k * kCrcThreads + t] = u32x4{w.s[k], w.s[k], w.s[k], w.s[k]};
    const uint32_t e = t >> 3, nib_table = e >> 4, nib = e & 15u;
    *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(lds + kCrcGnAt) + (nib_table >> 1) * 4096u + nib * 256u +
                              (nib_table & 1u) * 128u + (t & 7u) * 16u) =
        u32x4{w.advance, w.advance, w.advance, w.advance};
    lds[t] = w.behind;
}

// The workgroup's tables are written: wait for this wave's LDS writes and
// meet the other waves, without waiting for the record loads in flight (a
// __syncthreads would, and every wave would then start folding only when the
// slowest of the workgroup's first batches had landed).  The empty asm
// statements keep the compiler from moving memory accesses across.
__device__ __forceinline__ void crc_tables_ready() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left alone
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Groups of padding only (in stripe 0) are skipped, not folded: the registers are still zero there.
__device__ __forceinline__ int crc_lead(int64_t start) {
    return start < 0 ? static_cast<int>((-start) / kCrcGroup) : 0;
}

// Issue the loads of the first batch of the stripe of `groups` groups at record offset `start` into `a`.
// Chain c takes groups lead + c, lead + c + kCrcChains, ...  Only the first batch may hold front padding,
// and only the last may hold fewer groups than chains.
//
// Aligned records take one path without branches.  A chain past the stripe's groups loads the stripe's
// last group again, a word of front padding loads the record's first word, and crc_stripe_rest zeroes them
// once the loads have landed (crc_first_words_kept).  The host sends records of fewer than 16 bytes, or of
// 2 GiB or more, down the unaligned path, so every offset here is a record word's and fits 32 bits: the
// loads take the record's address from scalar registers and one 32-bit offset a chain from a vector
// register.  (With two load paths into the same registers the compiler waited for every earlier load, the
// table words' included, before issuing these, and HBM sat idle for the table words' round trip; zeroing
// here would wait for these loads before the tables are filled.)
// Only the first chain can hold padding (less than a group of it lies before the first group loaded).
__device__ __forceinline__ void crc_first_words_kept(int64_t start, int groups, uint32_t lane, u32x4* a) {
    const int g = crc_lead(start);
    const int count = groups - g < kCrcChains ? groups - g : kCrcChains;
#pragma unroll
    for (int c = 1; c < kCrcChains; ++c)
        if (c >= count) a[c] = u32x4{0u, 0u, 0u, 0u};  // wave-uniform
    const int64_t at = start + static_cast<int64_t>(g) * kCrcGroup;  // in (-1024, 2^31)
    if (static_cast<int>(lane) * kCrcRun < -static_cast<int>(at)) a[0] = u32x4{0u, 0u, 0u, 0u};
}

template <bool kAligned>
__device__ __forceinline__ void crc_stripe_first(const uint8_t* __restrict__ rec, int64_t start, int groups,
                                                 uint32_t lane, u32x4* a) {
    static_assert(kCrcRunWords == 1, "one word per chain and batch");
    const int g = crc_lead(start);
    const int count = groups - g < kCrcChains ? groups - g : kCrcChains;
    const int64_t at = start + static_cast<int64_t>(g) * kCrcGroup;
    if (!kAligned) {
        crc_load_any<false>(rec, at, count, lane, a);
        return;
    }
    const int at32 = static_cast<int>(at);  // in (-1024, 2^31)
    GlobalByte* base = crc_opaque(rec);  // in scalar registers (crc_opaque)
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c) {
        const int cc = c < count ? c : count - 1;
        int off = at32 + cc * kCrcGroup + static_cast<int>(lane) * kCrcRun;
        off = off < 0 ? 0 : off;
        a[c] = __builtin_nontemporal_load((GlobalWord*)(base + static_cast<uint32_t>(off)));
    }
}

// One wave's job: the raw CRC of the stripe of `groups` groups whose first byte is at record offset
// `start` (negative in the first stripe: front padding), the XOR of the wave's lanes.  The loads of its
// first batch into `a` were issued by crc_stripe_first, possibly before the tables were filled.
// The stripe's raw CRC from its chains' registers after `m` groups folded, the XOR of the wave's lanes.
// Horner over the chains in the order of their last groups: the chain whose last group is d groups before
// the stripe's end is (m - 1 - d) mod kCrcChains; chains that took no group hold zero.  Then each lane's
// register is shifted past the lanes after it.
__device__ __forceinline__ uint32_t crc_stripe_close(const uint32_t* lds, const uint32_t* acc, int m,
                                                     uint32_t lane_shift) {
    const uint32_t* behind_table = lds;
    uint32_t x = 0;
#pragma unroll
    for (int d = kCrcChains - 1; d >= 0; --d) {
        const int c = ((m - 1 - d) % kCrcChains + kCrcChains) % kCrcChains;  // wave-uniform
        uint32_t pick = acc[0];
#pragma unroll
        for (int k = 1; k < kCrcChains; ++k) pick = c == k ? acc[k] : pick;
        x = (d == kCrcChains - 1 ? 0u : crc_advance(behind_table, x)) ^ pick;
    }
    // The lane's constant is the same for every job: hidden from the compiler here, or it keeps the
    // multiply's 32 masks live across the job loop.
    uint32_t shift = lane_shift;
    asm volatile("" : "+v"(shift));
    x = gf_mul(shift, x);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    return x;
}

template <bool kAligned>
__device__ __forceinline__ uint32_t crc_stripe_rest(const uint32_t* lds, uint32_t lane, uint32_t cols,
                                                    uint32_t lane_shift, const uint8_t* __restrict__ rec,
                                                    int64_t start, int groups, u32x4* a) {
    const int lead = crc_lead(start);
    uint32_t acc[kCrcChains];
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c) acc[c] = 0;
    u32x4 b[kCrcBatchWords];
    int g = lead;
    const int count = groups - g < kCrcChains ? groups - g : kCrcChains;
    // The first batch's loads are complete before the steady state starts, which the wait for its
    // prefetches then counts on (vmcnt(0); expcnt and lgkmcnt left alone).
    __builtin_amdgcn_s_waitcnt(0x0F70);
    if (kAligned) crc_first_words_kept(start, groups, lane, a);
    while (true) {
        if (g + 2 * kCrcChains > groups) {
            crc_fold_rest<kAligned>(lds, cols, rec, start, groups, g, count, lane, a, acc);
            break;
        }
        crc_load_batch(rec, start + static_cast<int64_t>(g + kCrcChains) * kCrcGroup, lane, b);
        crc_fold_batch(lds, cols, a, acc, kCrcChains);
        g += kCrcChains;
        if (g + 2 * kCrcChains > groups) {
            crc_fold_rest<kAligned>(lds, cols, rec, start, groups, g, kCrcChains, lane, b, acc);
            break;
        }
        crc_load_batch(rec, start + static_cast<int64_t>(g + kCrcChains) * kCrcGroup, lane, a);
        crc_fold_batch(lds, cols, b, acc, kCrcChains);
        g += kCrcChains;
    }
    return crc_stripe_close(lds, acc, groups - lead, lane_shift);
}

// x^(8 * stripe_bytes * 2^i) mod P: the shifts of a stripe past the ones after it.
struct CrcStripePowers {
    uint32_t p[6];
};

__device__ __forceinline__ uint32_t crc_shift_stripes(const CrcStripePowers& powers, int behind, uint32_t x) {
#pragma unroll
    for (int i = 0; i < 6; ++i)
        if ((behind >> i) & 1) x = gf_mul(powers.p[i], x);
    return x;
}

// Jobs spread over the chip: the waves take (record, stripe) jobs in turn and
// write each stripe's raw CRC to `partial`; crc_combine_kernel then gives the
// records' CRC32C.  For few records, whose stripes must spread over many CUs.
template <bool kAligned>
__global__ __launch_bounds__(kCrcThreads) void crc_stripes_kernel(const uint8_t* __restrict__ records, uint64_t pitch,
                                                                 int64_t n_records, int64_t stripes, int groups,
                                                                 uint64_t pad, uint32_t* __restrict__ partial) {
    __shared__ uint32_t lds[(kCrcAdvanceBytes + kCrcPrivateBytes + kCrcBehindBytes) / 4];
    const uint32_t lane = threadIdx.x & 63u;
    // Jobs, records and stripes fit 32 bits (the host checks): 32-bit job arithmetic keeps the scalar
    // registers free of 64-bit division.
    const uint32_t jobs = static_cast<uint32_t>(n_records) * static_cast<uint32_t>(stripes);
    const uint32_t waves = gridDim.x * kCrcWaves;
    const int64_t stripe_bytes = static_cast<int64_t>(groups) * kCrcGroup;
    const uint32_t first = blockIdx.x * kCrcWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const auto job_record = [&](uint32_t job) {
        return records + static_cast<int64_t>(job / static_cast<uint32_t>(stripes)) * pitch;
    };
    const auto job_start = [&](uint32_t job) {
        return static_cast<int64_t>(job % static_cast<uint32_t>(stripes)) * stripe_bytes - static_cast<int64_t>(pad);
    };
    uint32_t lane_shift, cols;
    {
        // The table words are read first, then the first job's first batch, which is in flight while the
        // tables are filled.
        const CrcTableWords words = crc_table_words();
        lane_shift = g_crc_tables[kCrcLaneShift + lane];
        // Issued by every wave, a wave without a job loading job 0's: under a branch the compiler would
        // count these loads as maybe not issued and have the fill wait for them.
        u32x4 a[kCrcBatchWords];
        const uint32_t any = first < jobs ? first : 0;
        crc_stripe_first<kAligned>(job_record(any), job_start(any), groups, lane, a);
        crc_fill_tables(lds, words);
        cols = crc_columns(lane);
        crc_tables_ready();
        if (first < jobs) {
            const uint32_t x =
                crc_stripe_rest<kAligned>(lds, lane, cols, lane_shift, job_record(first), job_start(first), groups, a);
            if (lane == 0) partial[first] = x;
        }
    }
    for (uint32_t job = first + waves; job < jobs; job += waves) {
        u32x4 a[kCrcBatchWords];
        crc_stripe_first<kAligned>(job_record(job), job_start(job), groups, lane, a);
        const uint32_t x = crc_stripe_rest<kAligned>(lds, lane, cols, lane_shift, job_record(job), job_start(job),
                                                     groups, a);
        if (lane == 0) partial[job] = x;
    }
}

// A round's stripe: its raw CRC shifted past the `behind` stripes after it in the record (stripes <= 16),
// posted to the workgroup's LDS slot of wave `wave`.
__device__ __forceinline__ void crc_stripe_post(uint32_t* stripe_crc, uint32_t lane, int wave, int behind,
                                                const CrcStripePowers& powers, uint32_t x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if ((behind >> i) & 1) {
            uint32_t power = powers.p[i];
            asm volatile("" : "+s"(power));  // per round, as for the lane shift
            x = gf_mul(power, x);
        }
    }
    if (lane == 0) stripe_crc[wave] = x;
}

// The end of a round: once every wave has posted its stripe, one thread per record XORs the record's
// stripes and adds the initial value's term.
__device__ __forceinline__ void crc_round_combine(const uint32_t* stripe_crc, int stripes, int per_group,
                                                  int64_t base, int64_t n_records, uint32_t init_term,
                                                  uint32_t* __restrict__ out) {
    __syncthreads();
    if (threadIdx.x < static_cast<unsigned>(per_group) && base + threadIdx.x < n_records) {
        uint32_t x = 0;
        for (int k = 0; k < stripes; ++k) x ^= stripe_crc[threadIdx.x * stripes + k];
        out[base + threadIdx.x] = ~(init_term ^ x);
    }
    __syncthreads();
}

// Whole records per workgroup: a round gives `per_group` records' stripes to
// the workgroup's waves (wave w: record w / stripes, stripe w % stripes),
// each wave shifts its stripe's raw CRC to the record's end, and the
// workgroup XORs them in LDS, so no second launch combines them.  For many
// records (the chip fills with a few stripes each).
// One round of crc_records_kernel: the records from `base` on.  `a` holds the wave's first batch already
// in flight when `loaded`.
template <bool kAligned>
__device__ __forceinline__ void crc_records_round(const uint32_t* lds, uint32_t* stripe_crc, uint32_t lane,
                                                  uint32_t cols, uint32_t lane_shift, int wave,
                                                  const uint8_t* __restrict__ records, uint64_t pitch,
                                                  int64_t n_records, int stripes, int groups, uint64_t pad,
                                                  const CrcStripePowers& powers, uint32_t init_term,
                                                  uint32_t* __restrict__ out, int64_t base, u32x4* a, bool loaded) {
    const int per_group = kCrcWaves / stripes;
    const int rec_in_round = wave / stripes, j = wave - rec_in_round * stripes;
    const int64_t r = base + rec_in_round;
    if (rec_in_round < per_group && r < n_records) {  // wave-uniform
        // The wave's stripe is the same every round: hidden here, or what the compiler derives from it
        // stays live across rounds and the registers spill.
        int64_t start = static_cast<int64_t>(j) * groups * kCrcGroup - static_cast<int64_t>(pad);
        asm volatile("" : "+s"(start));
        if (!loaded) crc_stripe_first<kAligned>(records + r * pitch, start, groups, lane, a);
        const uint32_t x =
            crc_stripe_rest<kAligned>(lds, lane, cols, lane_shift, records + r * pitch, start, groups, a);
        crc_stripe_post(stripe_crc, lane, wave, stripes - 1 - j, powers, x);
    }
    crc_round_combine(stripe_crc, stripes, per_group, base, n_records, init_term, out);
}

template <bool kAligned>
__global__ __launch_bounds__(kCrcThreads) void crc_records_kernel(const uint8_t* __restrict__ records, uint64_t pitch,
                                                                 int64_t n_records, int stripes, int groups,
                                                                 uint64_t pad, CrcStripePowers powers,
                                                                 uint32_t init_term, uint32_t* __restrict__ out) {
    __shared__ uint32_t lds[(kCrcAdvanceBytes + kCrcPrivateBytes + kCrcBehindBytes) / 4];
    __shared__ uint32_t stripe_crc[kCrcWaves];
    const uint32_t lane = threadIdx.x & 63u;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int per_group = kCrcWaves / stripes;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * per_group;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * per_group;
    uint32_t lane_shift, cols;
    {
        // The table words are read first, then the first round's first batch, which is in flight while the
        // tables are filled.
        const CrcTableWords words = crc_table_words();
        lane_shift = g_crc_tables[kCrcLaneShift + lane];
        // Issued by every wave, a wave without a record this round loading record 0's stripe: under a branch
        // the compiler would count these loads as maybe not issued and have the fill wait for them.
        u32x4 a[kCrcBatchWords];
        const int rec_in_round = wave / stripes, j = wave - rec_in_round * stripes;
        const int64_t r = rec_in_round < per_group && first + rec_in_round < n_records ? first + rec_in_round : 0;
        crc_stripe_first<kAligned>(records + r * pitch,
                                   static_cast<int64_t>(j) * groups * kCrcGroup - static_cast<int64_t>(pad), groups,
                                   lane, a);
        crc_fill_tables(lds, words);
        cols = crc_columns(lane);
        crc_tables_ready();
        if (first < n_records)  // workgroup-uniform
            crc_records_round<kAligned>(lds, stripe_crc, lane, cols, lane_shift, wave, records, pitch, n_records,
                                        stripes, groups, pad, powers, init_term, out, first, a, true);
    }
    for (int64_t base = first + stride; base < n_records; base += stride) {
        u32x4 a[kCrcBatchWords];
        crc_records_round<kAligned>(lds, stripe_crc, lane, cols, lane_shift, wave, records, pitch, n_records,
                                    stripes, groups, pad, powers, init_term, out, base, a, false);
    }
}

// One wave per record: lane j shifts stripe j's raw CRC past the stripes after it, the wave XORs them, and
// lane 0 adds the initial value's term.
__global__ __launch_bounds__(256) void crc_combine_kernel(const uint32_t* __restrict__ partial, int64_t n_records,
                                                          int stripes, CrcStripePowers powers, uint32_t init_term,
                                                          uint32_t* __restrict__ out) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n_records) return;  // the whole wave
    uint32_t x = 0;
    if (lane < stripes) x = crc_shift_stripes(powers, stripes - 1 - lane, partial[r * stripes + lane]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if (lane == 0) out[r] = ~(init_term ^ x);
}

// ----------------------------------------------------------------- gather with CRC32C
//
// The save's gather into device records with every record's CRC32C folded in
// on the way: one HBM pass (a read and a write of the session) where the
// gather and the CRC32C kernel take two reads and a write.  It is the CRC32C
// records kernel above with its loads taken from the cache and each word
// written to its record once it has landed: the same stripes, chains, LDS
// tables, batches and per-workgroup combine.  For layouts whose spans are
// whole KiB (each 1 KiB group of a record lies in one span, so a wave's load
// of a group is one 1 KiB run of the cache):
//   group_bases[g] + block * group_pitches[g]   the source of record group g,
// the groups' table built once per layout on the host.  A record's front
// padding (the stripe plan's) is whole groups, which are skipped.

// The loads of the batch of record groups g, g + 1, ..., g + count - 1 (count >= 1) of `block` into v:
// chains past `count` load the last of them again (crc_gather_zero then zeroes them).  The group's source
// address is wave-uniform (scalar loads of the groups' table); lane l loads its 16 bytes.
__device__ __forceinline__ void crc_gather_load(const int64_t* __restrict__ group_bases,
                                                const int64_t* __restrict__ group_pitches, int64_t block, int g,
                                                int count, uint32_t lane, u32x4* v) {
    // The groups' table is constant while the kernel runs: read through the constant address space, its
    // entries are scalar loads.  Through a global pointer the compiler loaded one of them with a vector load,
    // and the wait for it drained the batch in flight.
    using Table = const __attribute__((address_space(4))) int64_t;
    Table* bases = (Table*)group_bases;
    Table* pitches = (Table*)group_pitches;
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c) {
        const int at = g + (c < count ? c : count - 1);
        const __amdgpu_buffer_rsrc_t buffer =
            crc_buffer(reinterpret_cast<const void*>(uniform64(static_cast<uint64_t>(bases[at] + block * pitches[at]))),
                       kCrcGroup);
        v[c] = __builtin_amdgcn_raw_buffer_load_b128(buffer, lane * kCrcRun, 0, kCrcLoadPolicy);
    }
}

__device__ __forceinline__ void crc_gather_zero(int count, u32x4* v) {
#pragma unroll
    for (int c = 1; c < kCrcChains; ++c)
        if (c >= count) v[c] = u32x4{0u, 0u, 0u, 0u};  // wave-uniform
}

// The landed batch's words to the record (groups g .. g + count - 1 at `record`).  Ordinary stores: the
// records are read again soon (the device-to-host copy, SHA-256), and a session of up to a few hundred MB
// stays in the last-level cache between.  Into buffers the cache does not hold, nontemporal stores ran
// alike (4.5-4.7 TB/s at a TP = 8 shard).
__device__ __forceinline__ void crc_gather_store(char* __restrict__ record, int g, int count, uint32_t lane,
                                                 const u32x4* v) {
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c)
        if (c < count)  // wave-uniform
            *reinterpret_cast<u32x4*>(record + static_cast<int64_t>(g + c) * kCrcGroup + lane * kCrcRun) = v[c];
}

// One wave's job: record groups [g, end) of `block` gathered into `record` and folded; the first batch
// was issued into `a` by crc_gather_load.  Returns the stripe's raw CRC (the XOR of the wave's lanes).
__device__ __forceinline__ uint32_t crc_gather_stripe(const uint32_t* lds, uint32_t lane, uint32_t cols,
                                                      uint32_t lane_shift, const int64_t* __restrict__ group_bases,
                                                      const int64_t* __restrict__ group_pitches, int64_t block,
                                                      char* __restrict__ record, int g, int end, u32x4* a) {
    const int m = end - g;
    uint32_t acc[kCrcChains];
#pragma unroll
    for (int c = 0; c < kCrcChains; ++c) acc[c] = 0;
    u32x4 b[kCrcBatchWords];
    int count = m < kCrcChains ? m : kCrcChains;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the first batch has landed (vmcnt(0))
    crc_gather_zero(count, a);
    while (true) {
        if (g + 2 * kCrcChains > end) {
            // a holds the last batch but one, or the last: store and fold it, then the rest (if any).
            crc_gather_store(record, g, count, lane, a);
            crc_fold_batch(lds, cols, a, acc, count);
            g += kCrcChains;
            if (g < end) {
                count = end - g;
                crc_gather_load(group_bases, group_pitches, block, g, count, lane, a);
                crc_gather_zero(count, a);
                crc_gather_store(record, g, count, lane, a);
                crc_fold_batch(lds, cols, a, acc, count);
            }
            break;
        }
        crc_gather_load(group_bases, group_pitches, block, g + kCrcChains, kCrcChains, lane, b);
        crc_gather_store(record, g, kCrcChains, lane, a);
        crc_fold_batch(lds, cols, a, acc, kCrcChains);
        g += kCrcChains;
        count = kCrcChains;
        if (g + 2 * kCrcChains > end) {
            crc_gather_store(record, g, count, lane, b);
            crc_fold_batch(lds, cols, b, acc, count);
            g += kCrcChains;
            if (g < end) {
                count = end - g;
                crc_gather_load(group_bases, group_pitches, block, g, count, lane, a);
                crc_gather_zero(count, a);
                crc_gather_store(record, g, count, lane, a);
                crc_fold_batch(lds, cols, a, acc, count);
            }
            break;
        }
        crc_gather_load(group_bases, group_pitches, block, g + kCrcChains, kCrcChains, lane, a);
        crc_gather_store(record, g, kCrcChains, lane, b);
        crc_fold_batch(lds, cols, b, acc, kCrcChains);
        g += kCrcChains;
    }
    return crc_stripe_close(lds, acc, m, lane_shift);
}

// Records `blocks` gathered to out + i * out_pitch, their CRC32C to crcs[i].  A record is `stripes` stripes
// of `groups` groups, the first `lead` groups of stripe 0 being padding; the workgroup takes 16 / stripes
// records a round (wave w: record w / stripes, stripe w % stripes), as crc_records_kernel does.
__global__ __launch_bounds__(kCrcThreads) void gather_crc_kernel(
    const int64_t* __restrict__ blocks, int64_t n_records, const int64_t* __restrict__ group_bases,
    const int64_t* __restrict__ group_pitches, int stripes, int groups, int lead, CrcStripePowers powers,
    uint32_t init_term, char* __restrict__ out, int64_t out_pitch, uint32_t* __restrict__ crcs) {
    __shared__ uint32_t lds[(kCrcAdvanceBytes + kCrcPrivateBytes + kCrcBehindBytes) / 4];
    __shared__ uint32_t stripe_crc[kCrcWaves];
    const uint32_t lane = threadIdx.x & 63u;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int per_group = kCrcWaves / stripes;
    const int rec_in_round = wave / stripes, j = wave - rec_in_round * stripes;
    // The wave's record groups, the same every round.
    const int g_begin = j == 0 ? 0 : j * groups - lead, g_end = (j + 1) * groups - lead;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * per_group;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * per_group;
    uint32_t lane_shift, cols;
    {
        // Table words, then the first round's first batch (every wave: one without a record loads record
        // 0's, so the compiler counts the loads as issued), in flight while the tables are filled.
        const CrcTableWords words = crc_table_words();
        lane_shift = g_crc_tables[kCrcLaneShift + lane];
        const bool mine = rec_in_round < per_group && first + rec_in_round < n_records;  // wave-uniform
        const int64_t r = mine ? first + rec_in_round : 0;
        u32x4 a[kCrcBatchWords];
        const int m = g_end - g_begin;
        crc_gather_load(group_bases, group_pitches, blocks[r], g_begin, m < kCrcChains ? m : kCrcChains, lane, a);
        crc_fill_tables(lds, words);
        cols = crc_columns(lane);
        crc_tables_ready();
        if (mine) {
            const uint32_t x = crc_gather_stripe(lds, lane, cols, lane_shift, group_bases, group_pitches, blocks[r],
                                                 out + r * out_pitch, g_begin, g_end, a);
            crc_stripe_post(stripe_crc, lane, wave, stripes - 1 - j, powers, x);
        }
        if (first < n_records)  // workgroup-uniform
            crc_round_combine(stripe_crc, stripes, per_group, first, n_records, init_term, crcs);
    }
    for (int64_t base = first + stride; base < n_records; base += stride) {
        const int64_t r = base + rec_in_round;
        if (rec_in_round < per_group && r < n_records) {  // wave-uniform
            const int m = g_end - g_begin;
            u32x4 a[kCrcBatchWords];
            crc_gather_load(group_bases, group_pitches, blocks[r], g_begin, m < kCrcChains ? m : kCrcChains, lane,
                            a);
            const uint32_t x = crc_gather_stripe(lds, lane, cols, lane_shift, group_bases, group_pitches, blocks[r],
                                                 out + r * out_pitch, g_begin, g_end, a);
            crc_stripe_post(stripe_crc, lane, wave, stripes - 1 - j, powers, x);
        }
        crc_round_combine(stripe_crc, stripes, per_group, base, n_records, init_term, crcs);
    }
}

// ----------------------------------------------------------------- restore with CRC32C
//
// The restore kernel's copy with each record's CRC32C computed from the bytes
// on their way through, so a checked restore costs one pass over the host
// link and none over HBM.  The host link is the bound (57 GB/s against the
// several TB/s the LDS lookups sustain), so the tables are shared, not one
// copy per lane as in the CRC kernel above.
//
// One wave per (block, span) job, jobs in the reference kernel's order.  Lane
// l takes the 16-byte slots l, l + 64, l + 128, ... of its span and folds
// them into acc, advancing acc by one row (64 slots, 1 KiB) per slot, so acc
// is the raw CRC of the lane's slots with the others as zeros, at its last
// slot.  With r = slots mod 64, that slot ends 16 * ((r - 1 - l) mod 64)
// bytes before the last slot of the span, whichever lanes own the short last
// row; M[k] = x^(128 k) moves it there.  A span of 8 bytes past its slots (a
// block size that is not even) has that word copied and folded by lane 0,
// after the others move past it by x^64.  The wave's XOR is the raw CRC of
// the span at its end, partial[job]; the finish kernel shifts every span to
// the end of its record.

constexpr int kCheckedUnroll = 8;                 // slots per lane per pass: 8 KiB per wave, 32 KiB per workgroup
constexpr int kCheckedAdvance = 0;                // G: advance by 1 KiB, [4][256]
constexpr int kCheckedSlicing = 1024;             // S: slicing-by-4, [4][256]
constexpr int kCheckedRowShift = 2048;            // M[64]: x^(128 k)
constexpr int kCheckedLdsWords = kCheckedRowShift + 64;
constexpr int kCheckedPowers = kCheckedLdsWords;  // x^(8 * 2^k), k < 48, read from global memory only
// x^(8 n) for n < 2^36 as three lookups: x^(8 j), x^(8 * 2^12 j) and x^(8 * 2^24 j), j < 4096.
constexpr int kCheckedPow0 = kCheckedPowers + 48, kCheckedPow1 = kCheckedPow0 + 4096,
              kCheckedPow2 = kCheckedPow1 + 4096;
constexpr int kCheckedTableWords = kCheckedPow2 + 4096;
constexpr uint64_t kCheckedMaxShift = uint64_t(1) << 36;

__device__ uint32_t g_crc_checked_tables[kCheckedTableWords];

__device__ __forceinline__ uint32_t crc_dword_shared(const uint32_t* s, uint32_t x) {
    return xor3(s[x & 0xFFu], s[256 + ((x >> 8) & 0xFFu)], s[512 + ((x >> 16) & 0xFFu)]) ^ s[768 + (x >> 24)];
}

__device__ __forceinline__ uint32_t crc_word_shared(const uint32_t* s, u32x4 v) {
    uint32_t c = crc_dword_shared(s, v.x);
    c = crc_dword_shared(s, c ^ v.y);
    c = crc_dword_shared(s, c ^ v.z);
    return crc_dword_shared(s, c ^ v.w);
}

// A 16-byte slot, as one dwordx4 access (kWide) or two 8-byte ones.
template <bool kWide>
__device__ __forceinline__ u32x4 load_slot(const char* p) {
    if (kWide) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t a = __builtin_nontemporal_load(q), b = __builtin_nontemporal_load(q + 1);
    return u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32), static_cast<uint32_t>(b),
                 static_cast<uint32_t>(b >> 32)};
}

template <bool kWide>
__device__ __forceinline__ void store_slot(char* p, u32x4 v) {
    if (kWide) {
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
        return;
    }
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    __builtin_nontemporal_store(static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32), q);
    __builtin_nontemporal_store(static_cast<uint64_t>(v.z) | (static_cast<uint64_t>(v.w) << 32), q + 1);
}

// s_waitcnt vmcnt(0): every vector memory access of the wave so far has
// completed (on gfx9 the counter covers stores too).
constexpr unsigned kWaitMemory = 0x0F70;

// Copy one span (nbytes a multiple of 8) with one wave, to `dst` and with
// kTwo also to `dst2`, and return this lane's share of its raw CRC32C at the
// span's end.  (Loading the next pass before folding this one measured no
// faster, into HBM or over the link, and slowed the TP = 8 shard's gather.)
//
// kPaced, for writes into pinned host memory: each slot's stores wait until
// the wave's earlier accesses have completed, so a wave has one slot's
// writes in flight.  Sixteen waves a CU issuing a whole pass of host writes
// at once queue more than the link drains, and the queue holds up other
// CUs' HBM traffic: a decode step beside such a save ran twice its time
// (p99 stall 1.45 ms, rotating fp8 workload); paced, 0.14 ms, and the save
// still fills its share of the link (41-44 GB/s on 4 workgroups).
template <bool kWide, bool kTwo, bool kPaced>
__device__ __forceinline__ uint32_t copy_span_crc(const char* __restrict__ src, char* __restrict__ dst,
                                                  char* __restrict__ dst2, int64_t nbytes, int lane,
                                                  const uint32_t* lds) {
    const uint32_t* slicing = lds + kCheckedSlicing;
    const int64_t slots = nbytes >> 4;
    uint32_t acc = 0;
    auto store = [&](int64_t at, const u32x4& v) {
        if (kPaced) __builtin_amdgcn_s_waitcnt(kWaitMemory);
        store_slot<kWide>(dst + at, v);
        if (kTwo) store_slot<kWide>(dst2 + at, v);
    };
    for (int64_t row = 0; row < slots; row += kCheckedUnroll * 64) {  // wave-uniform
        const int64_t i = row + lane;
        u32x4 v[kCheckedUnroll];
        if (row + kCheckedUnroll * 64 <= slots) {
#pragma unroll
            for (int u = 0; u < kCheckedUnroll; ++u) v[u] = load_slot<kWide>(src + 16 * (i + u * 64));
#pragma unroll
            for (int u = 0; u < kCheckedUnroll; ++u) store(16 * (i + u * 64), v[u]);
#pragma unroll
            for (int u = 0; u < kCheckedUnroll; ++u) acc = crc_advance(lds, acc) ^ crc_word_shared(slicing, v[u]);
        } else {
#pragma unroll
            for (int u = 0; u < kCheckedUnroll; ++u)
                v[u] = i + u * 64 < slots ? load_slot<kWide>(src + 16 * (i + u * 64)) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int u = 0; u < kCheckedUnroll; ++u)
                if (i + u * 64 < slots) store(16 * (i + u * 64), v[u]);
#pragma unroll
            for (int u = 0; u < kCheckedUnroll; ++u)
                if (i + u * 64 < slots) acc = crc_advance(lds, acc) ^ crc_word_shared(slicing, v[u]);
        }
    }
    const int r = static_cast<int>(slots & 63);
    uint32_t x = gf_mul(lds[kCheckedRowShift + ((r - 1 - lane) & 63)], acc);
    if (nbytes & 8) {
        x = gf_mul(g_crc_checked_tables[kCheckedPowers + 3], x);  // past the last 8 bytes: x^64
        if (lane == 0) {
            const uint64_t w = *reinterpret_cast<const uint64_t*>(src + 16 * slots);
            *reinterpret_cast<uint64_t*>(dst + 16 * slots) = w;
            if (kTwo) *reinterpret_cast<uint64_t*>(dst2 + 16 * slots) = w;
            x ^= crc_dword_shared(slicing, crc_dword_shared(slicing, static_cast<uint32_t>(w)) ^
                                               static_cast<uint32_t>(w >> 32));
        }
    }
    return x;
}

__global__ __launch_bounds__(kRestoreThreads) void restore_checked_kernel(
    const int64_t* __restrict__ sources, const int64_t* __restrict__ blocks, int64_t n_blocks,
    const int64_t* __restrict__ offs, const int64_t* __restrict__ bases, const int64_t* __restrict__ pitches,
    const int64_t* __restrict__ words, int64_t n_spans, uint32_t* __restrict__ partial) {
    __shared__ uint32_t lds[kCheckedLdsWords];
    for (int i = threadIdx.x; i < kCheckedLdsWords; i += kRestoreThreads) lds[i] = g_crc_checked_tables[i];
    __syncthreads();
    constexpr int kWaves = kRestoreThreads / 64;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int64_t jobs = n_blocks * n_spans;
    for (int64_t job = static_cast<int64_t>(blockIdx.x) * kWaves + wave; job < jobs;
         job += static_cast<int64_t>(gridDim.x) * kWaves) {
        const int64_t b = job / n_spans, s = job - b * n_spans;
        const char* src = reinterpret_cast<const char*>(sources[b] + offs[s]);
        char* dst = reinterpret_cast<char*>(bases[s] + blocks[b] * pitches[s]);
        const int64_t nbytes = words[s] * 8;
        const bool wide = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
        uint32_t x = wide ? copy_span_crc<true, false, false>(src, dst, nullptr, nbytes, lane, lds)
                          : copy_span_crc<false, false, false>(src, dst, nullptr, nbytes, lane, lds);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
        if (lane == 0) partial[job] = x;
    }
}

// The save's gather with the CRC32C folded in, the checked restore's inverse:
// one wave per (block, span) job copies the span from the cache to its record
// at dests[b] (pinned host memory over the link, or device memory) and, with
// kStage, also to stage + b * stage_pitch (device memory, for the SHA-256
// kernels), and leaves the span's raw CRC in partial[job] for
// restore_checked_finish_kernel.  One read of the cache gives the record, its
// device copy and its CRC32C.
//
// Over the host link (a small grid of whole CUs) a workgroup is 1024 lanes:
// one wave per SIMD waits out each pass's loads and folds, so sixteen keep a
// CU's share of the link busy (a direct hashed save of 4 such workgroups ran
// at 30 GB/s with 256-lane ones).  Into HBM (a full grid) it is 256 lanes.
constexpr int kGatherLinkThreads = 1024;

template <bool kStage, int kT>
__global__ __launch_bounds__(kT) void gather_checked_kernel(
    const int64_t* __restrict__ dests, const int64_t* __restrict__ blocks, int64_t n_blocks,
    const int64_t* __restrict__ offs, const int64_t* __restrict__ bases, const int64_t* __restrict__ pitches,
    const int64_t* __restrict__ words, int64_t n_spans, char* __restrict__ stage, int64_t stage_pitch,
    uint32_t* __restrict__ partial) {
    __shared__ uint32_t lds[kCheckedLdsWords];
    for (int i = threadIdx.x; i < kCheckedLdsWords; i += kT) lds[i] = g_crc_checked_tables[i];
    __syncthreads();
    constexpr int kWaves = kT / 64;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int64_t jobs = n_blocks * n_spans;
    for (int64_t job = static_cast<int64_t>(blockIdx.x) * kWaves + wave; job < jobs;
         job += static_cast<int64_t>(gridDim.x) * kWaves) {
        const int64_t b = job / n_spans, s = job - b * n_spans;
        const char* src = reinterpret_cast<const char*>(bases[s] + blocks[b] * pitches[s]);
        char* dst = reinterpret_cast<char*>(dests[b] + offs[s]);
        char* dst2 = kStage ? stage + b * stage_pitch + offs[s] : nullptr;
        const int64_t nbytes = words[s] * 8;
        const bool wide = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                            reinterpret_cast<uintptr_t>(dst2)) & 15) == 0;
        // Into pinned memory (the link-bound shape) the writes are paced; into HBM they are not.
        constexpr bool kPaced = kT == kGatherLinkThreads;
        uint32_t x = wide ? copy_span_crc<true, kStage, kPaced>(src, dst, dst2, nbytes, lane, lds)
                          : copy_span_crc<false, kStage, kPaced>(src, dst, dst2, nbytes, lane, lds);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
        if (lane == 0) partial[job] = x;
    }
}

// x^(8 n) mod P for n < 2^36: two multiplications of three table entries.
__device__ __forceinline__ uint32_t xpow8n(uint64_t n) {
    const uint32_t* t = g_crc_checked_tables;
    return gf_mul(gf_mul(t[kCheckedPow0 + (n & 4095u)], t[kCheckedPow1 + ((n >> 12) & 4095u)]),
                  t[kCheckedPow2 + ((n >> 24) & 4095u)]);
}

// Record r's CRC32C from its spans' partials: span j's raw CRC moves from the
// span's end to the record's, x^(8 (record_bytes - offset_j - bytes_j)), and
// the initial ~0 adds init_term.  The shifts (the same for every record) are
// the workgroup's first work, in dynamic LDS, one span per lane; then one
// wave per record, its lanes over the record's spans, XOR-reduced.
constexpr int kFinishThreads = 256;

__global__ __launch_bounds__(kFinishThreads) void restore_checked_finish_kernel(
    const uint32_t* __restrict__ partial, int64_t n_records, const int64_t* __restrict__ offs,
    const int64_t* __restrict__ words, int64_t n_spans, uint64_t record_bytes, uint32_t init_term,
    uint32_t* __restrict__ out) {
    extern __shared__ uint32_t shifts[];
    for (int64_t j = threadIdx.x; j < n_spans; j += kFinishThreads)
        shifts[j] = xpow8n(record_bytes - static_cast<uint64_t>(offs[j]) - static_cast<uint64_t>(words[j]) * 8);
    __syncthreads();
    constexpr int kWaves = kFinishThreads / 64;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int64_t wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * kWaves + wave; r < n_records;
         r += static_cast<int64_t>(gridDim.x) * kWaves) {
        uint32_t x = 0;
        for (int64_t j = lane; j < n_spans; j += 64) x ^= gf_mul(shifts[j], partial[r * n_spans + j]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
        if (lane == 0) out[r] = ~(init_term ^ x);
    }
}

// ----------------------------------------------------------------- SHA-256 (FIPS 180-4)
//
// SHA-256 is a sequential chain of 64-byte compressions within a record, so
// records are the only parallelism, and a few hundred records fill only a few
// dozen of the chip's 1024 SIMDs.  A record's time is therefore the time of
// its chain of rounds (a wave64 VALU instruction takes 4 cycles of its SIMD),
// and everything that does not depend on the chaining state is moved off it:
//   * two producer waves (one record per lane, alternate blocks of a step)
//     load each block a step ahead, byte-swap it, expand the message schedule
//     and add the round constants (W[t] + K[t]) into LDS;
//   * two round waves run only the 64 rounds, two lanes per record (the
//     e-half and the a-half of each round side by side, the a-half one round
//     behind; see sha_block), 10 VALU per round.
// Workgroup = two round waves + two producer waves over the same 64 records;
// the producers fill one half of a double buffer of kShaStep blocks while the
// round waves read the other.

__constant__ uint32_t kSha[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2,
};

__device__ __forceinline__ uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
__device__ __forceinline__ uint32_t bswap(uint32_t x) { return __builtin_bswap32(x); }

constexpr int kShaBlockQuads = 16;  // 64 schedule words per block, read 4 at a time
constexpr int kShaColumns = 65;     // 64 records, then {1,1,1,1} for the a-lanes

// Block `blk` of a record as 16 big-endian words, FIPS 180-4 padding included:
// blocks [0, whole) are payload, then 1 or 2 final blocks carry the tail,
// 0x80, zeros and the 64-bit bit length.
template <bool kAligned>
__device__ __forceinline__ void sha_message(const uint8_t* __restrict__ p, uint64_t record_bytes, uint64_t whole,
                                            int nfinal, uint64_t blk, uint32_t w[16]) {
    if (blk < whole) {
        const uint8_t* bp = p + 64 * blk;
        if (kAligned) {
            const u32x4* q = reinterpret_cast<const u32x4*>(bp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4 v = q[i];
                w[4 * i] = bswap(v.x);
                w[4 * i + 1] = bswap(v.y);
                w[4 * i + 2] = bswap(v.z);
                w[4 * i + 3] = bswap(v.w);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                w[i] = static_cast<uint32_t>(bp[4 * i]) << 24 | static_cast<uint32_t>(bp[4 * i + 1]) << 16 |
                       static_cast<uint32_t>(bp[4 * i + 2]) << 8 | static_cast<uint32_t>(bp[4 * i + 3]);
        }
        return;
    }
    const uint64_t rest = record_bytes - 64 * whole;
    const uint8_t* tail = p + 64 * whole;
    const uint64_t bits = record_bytes * 8;
    const int f = static_cast<int>(blk - whole);
    for (int i = 0; i < 16; ++i) {
        uint32_t word = 0;
        for (int k = 0; k < 4; ++k) {
            const uint64_t pos = static_cast<uint64_t>(64 * f + 4 * i + k);
            uint32_t byte = 0;
            if (pos < rest)
                byte = tail[pos];
            else if (pos == rest)
                byte = 0x80;
            else if (pos >= static_cast<uint64_t>(64 * nfinal - 8))
                byte = static_cast<uint32_t>(bits >> (8 * (64 * nfinal - 1 - pos))) & 0xFF;
            word |= byte << (24 - 8 * k);
        }
        w[i] = word;
    }
}

// Block `blk` as 16 words whose byte swaps are the message words: payload
// blocks of aligned records are the loaded words themselves, so the swap can
// wait until the loads have landed.
template <bool kAligned>
__device__ __forceinline__ void sha_message_raw(const uint8_t* __restrict__ p, uint64_t record_bytes, uint64_t whole,
                                                int nfinal, uint64_t blk, uint32_t raw[16]) {
    if (kAligned && blk < whole) {
        const u32x4* q = reinterpret_cast<const u32x4*>(p + 64 * blk);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 v = q[i];
            raw[4 * i] = v.x;
            raw[4 * i + 1] = v.y;
            raw[4 * i + 2] = v.z;
            raw[4 * i + 3] = v.w;
        }
        return;
    }
    uint32_t w[16];
    sha_message<kAligned>(p, record_bytes, whole, nfinal, blk, w);
#pragma unroll
    for (int i = 0; i < 16; ++i) raw[i] = bswap(w[i]);
}

// Producer: W[t] + K[t] for t = 0..63 into one LDS slot, [quad][lane].
__device__ __forceinline__ void sha_schedule(uint32_t w[16], u32x4 (*slot)[kShaColumns], int lane) {
#pragma unroll
    for (int q = 0; q < kShaBlockQuads; ++q) {
        uint32_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 4 * q + i;
            uint32_t wt;
            if (t < 16) {
                wt = w[t];
            } else {
                const uint32_t x15 = w[(t - 15) & 15], x2 = w[(t - 2) & 15];
                const uint32_t s0 = xor3(rotr(x15, 7), rotr(x15, 18), x15 >> 3);
                const uint32_t s1 = xor3(rotr(x2, 17), rotr(x2, 19), x2 >> 10);
                wt = w[t & 15] + s0 + w[(t - 7) & 15] + s1;
                w[t & 15] = wt;
            }
            v[i] = wt + kSha[t];
        }
        slot[q][lane] = u32x4{v[0], v[1], v[2], v[3]};
    }
}

// Round waves: two lanes per record.  Within each 8-lane half row, lanes 0-3
// are "e-lanes" holding (e, f, g, h) and lanes 4-7 "a-lanes" holding (a, b,
// c, d); e-lane i and a-lane 7 - i hold one record (DPP row_half_mirror
// swaps them).  Both halves run one instruction stream on registers X0..X3,
// the a-half two rounds behind: in slot t the e-lanes do round t and the
// a-lanes round t - 2.  A slot computes
//   W = (X3 ^ m) + K + partner's X1                   h + W[t]+K[t] + d | e' - d
//   S = rotr(X0, r1) ^ rotr(X0, r2) ^ rotr(X0, r3)    Sigma1(e) | Sigma0(a)
//   u = m ? ~(X0 ^ X1) : X0;  C = u ? X1 : X2         Ch(e,f,g) | Maj(a,b,c)
//   X0' = S + C + W                                    e' = d + T1 | a' = T1 + T2
// with m = 0 and K = W[t]+K[t] on e-lanes, m = ~0 and K = 1 on a-lanes
// (Maj(a,b,c) = ~(a^b) ? b : c bitwise; ~d + 1 = -d).  With the two-round
// lag the partner's X1 is what each half needs: the a-lanes' X1 is a of
// round t - 4, the e-lanes' d; the e-lanes' X1 is e' of round t - 2, the
// round the a-lanes are on.  So one DPP add serves both halves, it reads a
// register written two slots before, and a slot is 9 VALU whose only chain
// is the rotations (or Ch/Maj) into one add3.  (Both halves on the same
// round need a DPP add on the chain and a second one for d: 11 issue slots
// a round against 9.)
constexpr int kDppIdentity = 0xE4;    // quad_perm [0,1,2,3]: lane i reads itself
constexpr int kDppHalfMirror = 0x141;  // lane i reads lane 7 - i of its half row
constexpr int kEBanks = 0x5, kABanks = 0xA;

struct ShaHalf {
    uint32_t r1, r2, r3, m;
};

__device__ __forceinline__ uint32_t rotr_v(uint32_t x, uint32_t n) { return __builtin_amdgcn_alignbit(x, x, n); }
// An empty asm operand: the compiler must treat x as an unknown register value
// from here on (no constant folding of lane masks, no reassociating sums).
__device__ __forceinline__ void opaque(uint32_t& x) { asm("" : "+v"(x)); }

template <int kCtrl, int kBanks>
__device__ __forceinline__ uint32_t dpp_bits(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, 0xF, kBanks, false));
}
// The partner's x.
__device__ __forceinline__ uint32_t from_partner(uint32_t x) { return dpp_bits<kDppHalfMirror, 0xF>(x); }
// The partner's x on e-lanes (from the a-lane), 0 on a-lanes; and the other way round.
__device__ __forceinline__ uint32_t from_a_partner(uint32_t x) { return dpp_bits<kDppHalfMirror, kEBanks>(x); }
__device__ __forceinline__ uint32_t from_e_partner(uint32_t x) { return dpp_bits<kDppHalfMirror, kABanks>(x); }
// x on e-lanes, 0 on a-lanes; and the other way round.
__device__ __forceinline__ uint32_t on_e_lanes(uint32_t x) { return dpp_bits<kDppIdentity, kEBanks>(x); }
__device__ __forceinline__ uint32_t on_a_lanes(uint32_t x) { return dpp_bits<kDppIdentity, kABanks>(x); }

__device__ __forceinline__ uint32_t quad_word(const u32x4& q, int t) {
    return (t & 3) == 0 ? q.x : (t & 3) == 1 ? q.y : (t & 3) == 2 ? q.z : q.w;
}

// Two-lane state between slots: X0..X3 as above and the chaining value, held
// as E (the e-lanes' words) and F (the a-lanes' words).
struct ShaLanes {
    uint32_t x[4];
    uint32_t e[4], f[4];
};

__device__ __forceinline__ uint32_t sha_sigma(uint32_t x0, const ShaHalf& k) {
    return xor3(rotr_v(x0, k.r1), rotr_v(x0, k.r2), rotr_v(x0, k.r3));
}

// bitop3 tables index bits as (src0 << 2) | (src1 << 1) | src2.
__device__ __forceinline__ uint32_t sha_choose(uint32_t x0, uint32_t x1, uint32_t x2, const ShaHalf& k) {
    const uint32_t u = __builtin_amdgcn_bitop3_b32(x0, x1, k.m, 0xD2);  // m ? ~(x0 ^ x1) : x0
    return __builtin_amdgcn_bitop3_b32(x1, x2, u, 0xE4);                // u ? x1 : x2
}

// One slot whose W has been summed but for S + C.
__device__ __forceinline__ void sha_slot_finish(ShaLanes& l, uint32_t w, const ShaHalf& k) {
    const uint32_t v = sha_sigma(l.x[0], k) + sha_choose(l.x[0], l.x[1], l.x[2], k) + w;
    l.x[3] = l.x[2]; l.x[2] = l.x[1]; l.x[1] = l.x[0]; l.x[0] = v;
}

// A slot inside a block: one DPP add for both halves.
__device__ __forceinline__ void sha_slot(ShaLanes& l, uint32_t word, const ShaHalf& k) {
    uint32_t w = (l.x[3] ^ k.m) + word;
    opaque(w);
    w = from_partner(l.x[1]) + w;
    opaque(w);
    sha_slot_finish(l, w, k);
}

// Slot 0 or 1 of a block: the e-lanes' rounds 0 and 1 of this block, the
// a-lanes' rounds 62 and 63 of the previous one.  The e-lanes have fed
// forward (their X holds this block's state) and the a-lanes have not: the
// e-lanes' d is the a-lanes' X1 plus the chaining word not yet added (`fw`,
// d then c), and the a-lanes' e' is the e-lanes' X1 before the feed-forward
// (`unfed`: the slot before's X1 and X0).
__device__ __forceinline__ void sha_slot_turn(ShaLanes& l, uint32_t word, uint32_t fw, uint32_t unfed,
                                              const ShaHalf& k) {
    uint32_t w = (l.x[3] ^ k.m) + word;
    opaque(w);
    w = from_a_partner(l.x[1] + fw) + w;
    opaque(w);
    w = from_e_partner(unfed) + w;
    opaque(w);
    sha_slot_finish(l, w, k);
}

// Between blocks: the e-lanes add their chaining words to X0..X3 and keep the
// sums as the chaining words (a-lanes untouched); slots 0 and 1 finish the
// previous block on the a-lanes, which then do the same with F.
__device__ __forceinline__ void sha_block_turn(ShaLanes& l, uint32_t word0, uint32_t word1, const ShaHalf& k) {
    const uint32_t unfed0 = l.x[0], unfed1 = l.x[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) l.e[i] = l.x[i] = l.x[i] + on_e_lanes(l.e[i]);
    sha_slot_turn(l, word0, l.f[3], unfed1, k);
    sha_slot_turn(l, word1, l.f[2], unfed0, k);
#pragma unroll
    for (int i = 0; i < 4; ++i) l.f[i] = l.x[i] = l.x[i] + on_a_lanes(l.f[i]);
}

// The W+K words come from LDS in batches of four 16-byte quads (16 rounds),
// each batch read a whole batch ahead of its use and waited for with one
// s_waitcnt: a wait costs a wave about 7 cycles however little it waits, so
// one wait for 16 rounds rather than one for every 4.  A scheduling barrier
// after the reads keeps them where they are issued; left to itself the
// compiler sinks them to their first use, a batch later.
constexpr int kShaBatch = 4;                                 // quads a batch
constexpr int kShaBatches = kShaBlockQuads / kShaBatch;      // batches a block
constexpr unsigned kWaitLds = 0xC07F;                        // s_waitcnt lgkmcnt(0)

__device__ __forceinline__ void sha_read_batch(u32x4 dst[kShaBatch], const u32x4 (*slot)[kShaColumns], int batch,
                                               int column) {
#pragma unroll
    for (int j = 0; j < kShaBatch; ++j) dst[j] = slot[kShaBatch * batch + j][column];
    __builtin_amdgcn_sched_barrier(0);
}

// One block.  On entry the e-lanes hold the state after the previous block's
// round 63 and the a-lanes after its round 61 (see sha_block_turn), and q[0]
// holds this block's first W+K batch, not yet waited for; q[1] is free.  With
// kNext the first batch of `next` is read during the last batch, into q[0].
template <bool kNext>
__device__ __forceinline__ void sha_block(ShaLanes& l, u32x4 (&q)[2][kShaBatch], const u32x4 (*slot)[kShaColumns],
                                          const u32x4 (*next)[kShaColumns], int column, const ShaHalf& k) {
#pragma unroll
    for (int b = 0; b < kShaBatches; ++b) {
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        if (b + 1 < kShaBatches)
            sha_read_batch(q[(b + 1) & 1], slot, b + 1, column);
        else if (kNext)
            sha_read_batch(q[(b + 1) & 1], next, 0, column);
        const u32x4* cur = q[b & 1];
#pragma unroll
        for (int t = 16 * b; t < 16 * b + 16; ++t) {
            if (t == 0)
                sha_block_turn(l, quad_word(cur[0], 0), quad_word(cur[0], 1), k);
            else if (t > 1)
                sha_slot(l, quad_word(cur[(t >> 2) & 3], t), k);
        }
    }
}

// The lanes' state before the first block of a launch, from chaining value
// h[4] (the e-lanes' (e, f, g, h) or the a-lanes' (a, b, c, d)).  E = F = 0
// makes the first feed-forwards copies.  The a-lanes have no rounds 62 and
// 63 to finish, so they start as (c, d, y2, y3) with y3 and y2 chosen so that
// slots 0 and 1 yield b and then a: slot 0 computes Sigma0(c) + Maj(c, d, y2)
// + f - y3 and slot 1 Sigma0(b) + Maj(b, c, d) + e - y2, e and f being the
// partner's X0 and X1 before the (here empty) feed-forward.  After them the
// a-lanes hold (a, b, c, d).
__device__ __forceinline__ ShaLanes sha_lanes_start(const uint32_t h[4], bool a_lane, const ShaHalf& k) {
    ShaLanes l;
    const uint32_t y2 = sha_sigma(h[1], k) + sha_choose(h[1], h[2], h[3], k) + from_e_partner(h[0]) - h[0];
    const uint32_t y3 = sha_sigma(h[2], k) + sha_choose(h[2], h[3], y2, k) + from_e_partner(h[1]) - h[1];
    l.x[0] = a_lane ? h[2] : h[0];
    l.x[1] = a_lane ? h[3] : h[1];
    l.x[2] = a_lane ? y2 : h[2];
    l.x[3] = a_lane ? y3 : h[3];
#pragma unroll
    for (int i = 0; i < 4; ++i) l.e[i] = l.f[i] = 0;
    return l;
}

// After the last block: the e-lanes feed forward, the a-lanes run their
// rounds 62 and 63 (K = 1) and feed forward; the chaining value is E on
// e-lanes, F on a-lanes.
__device__ __forceinline__ void sha_lanes_finish(ShaLanes& l, bool a_lane, const ShaHalf& k, uint32_t h[4]) {
    sha_block_turn(l, 1u, 1u, k);
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = a_lane ? l.f[i] : l.e[i];
}

constexpr int kShaRoundWaves = 2;                  // round waves per workgroup, 32 records each
constexpr int kShaProducers = 2;                   // message-schedule waves, alternate blocks of a step
constexpr int kShaRecords = 32 * kShaRoundWaves;   // records per workgroup
constexpr int kShaThreads = 64 * (kShaRoundWaves + kShaProducers);  // the round waves, then the producers
constexpr int kShaStep = 4;  // blocks per barrier; the producers fill one half while the rounds read the other
constexpr int kShaProducerBlocks = kShaStep / kShaProducers;  // blocks of a step per producer

// A producer's step for block `blk` (of blocks below `end`): expand the words
// loaded for it, then start the loads of block blk + kShaAheadSteps *
// kShaStep into the same registers.  A producer keeps kShaAheadSteps register
// sets per block of a step, so each block's loads are in flight for two whole
// steps (about 10 us) before its expansion: beside a restore kernel's reads
// of host memory, loads issued one step ahead came back late and the round
// waves waited at the step barrier (58 cycles a round against 45).
constexpr int kShaAheadSteps = 2;

template <bool kAligned>
__device__ __forceinline__ void sha_produce(const uint8_t* __restrict__ p, uint64_t record_bytes, uint64_t whole,
                                            int nfinal, uint64_t end, uint64_t blk, uint32_t raw[16],
                                            u32x4 (*slot)[kShaColumns], int lane) {
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = bswap(raw[i]);
    const uint64_t next = blk + kShaAheadSteps * kShaStep;
    if (next < end) sha_message_raw<kAligned>(p, record_bytes, whole, nfinal, next, raw);
    sha_schedule(w, slot, lane);
}

// The register sets of the next two steps' blocks trade places.
__device__ __forceinline__ void sha_rotate_sets(uint32_t (&raw)[kShaAheadSteps][kShaProducerBlocks][16]) {
    static_assert(kShaAheadSteps == 2, "two sets");
#pragma unroll
    for (int j = 0; j < kShaProducerBlocks; ++j)
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint32_t t = raw[0][j][k];
            raw[0][j][k] = raw[1][j][k];
            raw[1][j][k] = t;
        }
}

using ShaSchedule = u32x4[2][kShaStep][kShaBlockQuads][kShaColumns];

// Blocks [b0, b1) of the chains of the `group`-th kShaRecords records.  b0 =
// 0 starts from the FIPS 180-4 initial value, otherwise from `state` (8 words
// per record, as a previous launch left them); b1 = nblocks writes the digest
// to `out`, otherwise the chaining state back to `state`.  A whole hash in
// one launch holds its stream (and any stream sharing its hardware queue) for
// the whole chain; the host can run it as a series of shorter launches.
template <bool kAligned>
__device__ __forceinline__ void sha256_group(ShaSchedule& sched, const uint8_t* __restrict__ records,
                                             uint64_t record_bytes, uint64_t pitch, int64_t n_records, uint64_t b0,
                                             uint64_t b1, uint32_t* __restrict__ state, uint32_t* __restrict__ out,
                                             int64_t group) {
    const int wave = threadIdx.x >> 6;
    const bool producer = wave >= kShaRoundWaves;
    const int part = wave - kShaRoundWaves;  // a producer's blocks of a step: part, part + kShaProducers, ...
    const int lane = threadIdx.x & 63;
    const bool a_lane = (lane >> 2) & 1;
    // Record of this lane within the workgroup's kShaRecords (producer lanes past them idle).
    // Round lanes: e-lane i and a-lane 7 - i of each 8-lane half row share a record.
    const int rec = producer ? lane
                             : wave * 32 + (lane >> 3) * 4 + (a_lane ? 3 - (lane & 3) : (lane & 3));
    const int64_t r = group * kShaRecords + rec;
    const bool live = rec < kShaRecords && r < n_records;
    // Lanes past the last record hash record 0 (in bounds) and store nothing.
    const uint8_t* p = records + (live ? r : 0) * pitch;
    const uint64_t whole = record_bytes / 64;
    const int nfinal = record_bytes - 64 * whole + 9 <= 64 ? 1 : 2;
    const uint64_t nblocks = whole + nfinal;
    const uint64_t span = b1 - b0;
    const uint64_t steps = (span + kShaStep - 1) / kShaStep;
    // raw[0]: the words of the producer's blocks of the next step to expand; raw[1]: of the step after.
    uint32_t raw[kShaAheadSteps][kShaProducerBlocks][16];
    if (producer) {
        for (int i = lane + 64 * part; i < 2 * kShaStep * kShaBlockQuads; i += 64 * kShaProducers) {
            const int slot = i / kShaBlockQuads;
            sched[slot / kShaStep][slot % kShaStep][i % kShaBlockQuads][64] = u32x4{1u, 1u, 1u, 1u};
        }
#pragma unroll
        for (int a = 0; a < kShaAheadSteps; ++a)
#pragma unroll
            for (int j = 0; j < kShaProducerBlocks; ++j) {
                const uint64_t i = static_cast<uint64_t>(a * kShaStep + part + kShaProducers * j);
                if (i < span) sha_message_raw<kAligned>(p, record_bytes, whole, nfinal, b0 + i, raw[a][j]);
            }
#pragma unroll
        for (int j = 0; j < kShaProducerBlocks; ++j) {
            const int i = part + kShaProducers * j;
            if (static_cast<uint64_t>(i) < span)
                sha_produce<kAligned>(p, record_bytes, whole, nfinal, b1, b0 + i, raw[0][j], sched[0][i], lane);
        }
        sha_rotate_sets(raw);
    }
    __syncthreads();
    ShaHalf half = a_lane ? ShaHalf{2, 13, 22, ~0u} : ShaHalf{6, 11, 25, 0u};
    opaque(half.m);
    uint32_t h[4];
    uint32_t* chain = state ? state + 8 * (live ? r : 0) + (a_lane ? 0 : 4) : nullptr;
    if (b0 > 0) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(chain);
        h[0] = v.x; h[1] = v.y; h[2] = v.z; h[3] = v.w;
    } else if (a_lane) {
        h[0] = 0x6a09e667; h[1] = 0xbb67ae85; h[2] = 0x3c6ef372; h[3] = 0xa54ff53a;
    } else {
        h[0] = 0x510e527f; h[1] = 0x9b05688c; h[2] = 0x1f83d9ab; h[3] = 0x5be0cd19;
    }
    ShaLanes l = sha_lanes_start(h, a_lane, half);
    const int column = a_lane ? 64 : rec;
    u32x4 q[2][kShaBatch];  // W+K batches, read into alternately
    for (uint64_t step = 0; step < steps; ++step) {
        const uint64_t first = b0 + step * kShaStep;
        if (producer) {
#pragma unroll
            for (int j = 0; j < kShaProducerBlocks; ++j) {
                const int i = part + kShaProducers * j;
                if (first + kShaStep + i < b1)
                    sha_produce<kAligned>(p, record_bytes, whole, nfinal, b1, first + kShaStep + i, raw[0][j],
                                          sched[(step + 1) & 1][i], lane);
            }
            sha_rotate_sets(raw);
        } else {
            sha_read_batch(q[0], sched[step & 1][0], 0, column);
#pragma unroll
            for (int i = 0; i < kShaStep; ++i) {
                if (first + i >= b1) break;
                if (i + 1 < kShaStep)
                    sha_block<true>(l, q, sched[step & 1][i], sched[step & 1][i + 1], column, half);
                else
                    sha_block<false>(l, q, sched[step & 1][i], nullptr, column, half);
            }
        }
        __syncthreads();
    }
    if (!producer) {
        sha_lanes_finish(l, a_lane, half, h);
        if (live) {
            if (b1 == nblocks)
                *reinterpret_cast<u32x4*>(out + 8 * r + (a_lane ? 0 : 4)) =
                    u32x4{bswap(h[0]), bswap(h[1]), bswap(h[2]), bswap(h[3])};
            else
                *reinterpret_cast<u32x4*>(chain) = u32x4{h[0], h[1], h[2], h[3]};
        }
    }
}

template <bool kAligned>
__global__ __launch_bounds__(kShaThreads) void sha256_kernel(const uint8_t* __restrict__ records,
                                                             uint64_t record_bytes, uint64_t pitch,
                                                             int64_t n_records, uint64_t b0, uint64_t b1,
                                                             uint32_t* __restrict__ state,
                                                             uint32_t* __restrict__ out) {
    __shared__ ShaSchedule sched;
    sha256_group<kAligned>(sched, records, record_bytes, pitch, n_records, b0, b1, state, out, blockIdx.x);
}

// Several independent ranges in one launch: range blockIdx.y, its blockIdx.x-th
// group of records.  Saves hashing at the same time share each launch, so
// they hash side by side on one stream (and one hardware queue) instead of in
// turn.
constexpr int kShaMaxRanges = 8;

struct ShaRange {
    const uint8_t* records;
    uint64_t record_bytes, pitch;
    int64_t n_records;
    uint64_t b0, b1;
    uint32_t* state;
    uint32_t* out;
};

struct ShaRanges {
    ShaRange r[kShaMaxRanges];
};

template <bool kAligned>
__global__ __launch_bounds__(kShaThreads) void sha256_ranges_kernel(ShaRanges ranges) {
    __shared__ ShaSchedule sched;
    const ShaRange& g = ranges.r[blockIdx.y];
    if (static_cast<int64_t>(blockIdx.x) * kShaRecords >= g.n_records) return;  // the whole workgroup
    sha256_group<kAligned>(sched, g.records, g.record_bytes, g.pitch, g.n_records, g.b0, g.b1, g.state, g.out,
                           blockIdx.x);
}

// The round's own issue rate, measured: one wave runs `reps` slots of the
// round waves' instruction sequence (sha_slot, both halves) on values seeded
// per lane, with no LDS, no waits and no barrier, between two reads of the
// shader clock (s_memtime) and of the 100 MHz constant clock (s_memrealtime).
// out[0] = shader cycles, out[1] = constant-clock ticks, out[2] = a checksum
// of the lanes' state (so the slots are not optimised away).
constexpr int kShaProbeUnroll = 16;

__global__ __launch_bounds__(64) void sha_round_probe_kernel(uint32_t seed, int reps, uint64_t* __restrict__ out) {
    const int lane = threadIdx.x;
    const bool a_lane = (lane >> 2) & 1;
    ShaHalf half = a_lane ? ShaHalf{2, 13, 22, ~0u} : ShaHalf{6, 11, 25, 0u};
    opaque(half.m);
    ShaLanes l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        l.x[i] = seed * 0x9E3779B9u + static_cast<uint32_t>(lane * 4 + i) * 0x85EBCA6Bu;
        l.e[i] = l.f[i] = 0;
    }
    uint32_t word = a_lane ? 1u : seed ^ 0x5A827999u;
    opaque(word);
    const int rounds = reps / kShaProbeUnroll;
#pragma unroll
    for (int i = 0; i < 4; ++i) opaque(l.x[i]);
    const uint64_t c0 = __builtin_amdgcn_s_memtime();
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
        for (int k = 0; k < kShaProbeUnroll; ++k) sha_slot(l, word, half);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) opaque(l.x[i]);
    const uint64_t c1 = __builtin_amdgcn_s_memtime();
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    uint32_t sum = l.x[0] ^ l.x[1] ^ l.x[2] ^ l.x[3];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum ^= __shfl_xor(sum, o);
    if (lane == 0) {
        out[0] = c1 - c0;
        out[1] = t1 - t0;
        out[2] = sum;
    }
}

// The chip's read rate at a given size, measured: the CRC32C kernels' shape
// (one 1024-lane workgroup a CU) reading `words` 16-byte words with
// nontemporal loads, four in flight per lane, and nothing else.  Each wave
// XORs what it read into one word of sink (16 a workgroup), so the XOR of
// sink is the XOR of the buffer's 32-bit words.
constexpr int kReadProbeLanes = 1024, kReadProbeUnroll = 4, kReadProbeGroups = 256;

__global__ __launch_bounds__(kReadProbeLanes) void read_probe_kernel(const u32x4* __restrict__ src, uint64_t words,
                                                                      uint32_t* __restrict__ sink) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kReadProbeLanes * kReadProbeUnroll;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * kReadProbeLanes * kReadProbeUnroll + threadIdx.x;
    u32x4 acc = {0, 0, 0, 0};
    for (; i + (kReadProbeUnroll - 1) * kReadProbeLanes < words; i += stride) {
        u32x4 v[kReadProbeUnroll];
#pragma unroll
        for (int u = 0; u < kReadProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * kReadProbeLanes);
#pragma unroll
        for (int u = 0; u < kReadProbeUnroll; ++u) acc ^= v[u];
    }
#pragma unroll
    for (int u = 0; u < kReadProbeUnroll; ++u)
        if (i + u * kReadProbeLanes < words) acc ^= src[i + u * kReadProbeLanes];
    uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (kReadProbeLanes / 64) + threadIdx.x / 64] = x;
}

// The chip's rate for a contiguous copy of a given size, measured: the pieces
// kernels' shape (one 64-lane workgroup a KiB, one nontemporal 16-byte load
// and store a lane) with no tables, no spans and no scattered side.
__global__ __launch_bounds__(64) void copy_probe_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                        uint64_t words) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (i < words) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// ----------------------------------------------------------------- host helpers

uint32_t host_gf_mul(uint32_t a, uint32_t b) {
    uint32_t p = 0;
    for (int i = 0; i < 32; ++i) {
        if ((a >> (31 - i)) & 1u) p ^= b;
        b = (b >> 1) ^ (kPoly & (0u - (b & 1u)));
    }
    return p;
}

// x^(8n) mod P, by squaring from x^(2^k).
uint32_t host_xpow8n(uint64_t n) {
    uint32_t sq = 0x40000000u;  // x^1
    uint32_t result = 0x80000000u;  // x^0
    uint64_t e = n * 8;
    while (e) {
        if (e & 1) result = host_gf_mul(sq, result);
        sq = host_gf_mul(sq, sq);
        e >>= 1;
    }
    return result;
}

uint32_t host_shift(uint32_t s, uint64_t nbytes) { return host_gf_mul(host_xpow8n(nbytes), s); }

std::mutex g_table_mutex;
bool g_tables_ready[64];

void ensure_crc_tables() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64)
        throw std::runtime_error("no current HIP device for the CRC32C tables");
    std::lock_guard<std::mutex> lock(g_table_mutex);
    if (g_tables_ready[device]) return;
    static uint32_t tables[kCrcTableWords];
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t m = host_xpow8n(4 - i);
        for (uint32_t v = 0; v < 256; ++v) tables[256 * i + v] = host_gf_mul(m, v);
    }
    const uint32_t advance = host_xpow8n(static_cast<uint64_t>(kCrcChains) * kCrcGroup);
    for (uint32_t i = 0; i < 8; ++i)
        for (uint32_t v = 0; v < 16; ++v) tables[kCrcAdvance + 16 * i + v] = host_gf_mul(advance, v << (4 * i));
    const uint32_t behind = host_xpow8n(kCrcGroup);
    for (uint32_t k = 0; k < 4; ++k)
        for (uint32_t v = 0; v < 256; ++v) tables[kCrcBehind + 256 * k + v] = host_gf_mul(behind, v << (8 * k));
    for (uint32_t l = 0; l < 64; ++l) tables[kCrcLaneShift + l] = host_xpow8n(static_cast<uint64_t>(kCrcRun) * (63 - l));
    hipError_t rc = hipMemcpyToSymbol(HIP_SYMBOL(g_crc_tables), tables, sizeof tables, 0, hipMemcpyHostToDevice);
    if (rc != hipSuccess) throw std::runtime_error(std::string("CRC32C table upload: ") + hipGetErrorString(rc));
    // The checked restore's: G (advance by one 1 KiB row), S (slicing-by-4), M, then x^(8 * 2^k).
    static uint32_t checked[kCheckedTableWords];
    const uint32_t row_shift = host_xpow8n(1024);
    for (uint32_t k = 0; k < 4; ++k)
        for (uint32_t v = 0; v < 256; ++v) {
            checked[kCheckedAdvance + 256 * k + v] = host_gf_mul(row_shift, v << (8 * k));
            checked[kCheckedSlicing + 256 * k + v] = tables[256 * k + v];
        }
    for (uint32_t k = 0; k < 64; ++k) checked[kCheckedRowShift + k] = host_xpow8n(16ull * k);
    for (uint32_t k = 0; k < 48; ++k) checked[kCheckedPowers + k] = host_xpow8n(1ull << k);
    const uint32_t steps[3] = {host_xpow8n(1), host_xpow8n(1ull << 12), host_xpow8n(1ull << 24)};
    for (int t = 0; t < 3; ++t) {
        uint32_t* table = checked + kCheckedPow0 + 4096 * t;
        table[0] = 0x80000000u;  // x^0
        for (uint32_t j = 1; j < 4096; ++j) table[j] = host_gf_mul(table[j - 1], steps[t]);
    }
    rc = hipMemcpyToSymbol(HIP_SYMBOL(g_crc_checked_tables), checked, sizeof checked, 0, hipMemcpyHostToDevice);
    if (rc != hipSuccess) throw std::runtime_error(std::string("CRC32C table upload: ") + hipGetErrorString(rc));
    g_tables_ready[device] = true;
}

template <typename F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        kvsnap::set_error(e.what());
        return -1;
    }
}

void check_launch(const char* what) {
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) throw std::runtime_error(std::string(what) + " launch: " + hipGetErrorString(rc));
}

// Longest hold: about 0.1 s at 2.4 GHz.
constexpr int kMaxHoldIters = 30000;

// The checked restore's finish keeps one shift per span in LDS.
constexpr int64_t kMaxCheckedSpans = 8192;

unsigned grid_for(int64_t jobs, int programs) {
    int64_t grid = programs > 0 ? (programs < jobs ? programs : jobs) : jobs;
    if (grid > (int64_t(1) << 30)) grid = int64_t(1) << 30;
    return static_cast<unsigned>(grid);
}

// A copy launch's shape: lanes per (block, span) job as a shift, and the grid.
// A group of lanes keeps `unroll` 16-byte loads per lane in flight while its
// span has at least twice that many vectors; shorter spans get fewer lanes,
// never less than a wave.  min_span_bytes <= 0 (unknown) keeps whole
// workgroups.  The shape never changes what is copied, only how fast.
struct CopyShape {
    int lane_shift;
    unsigned grid;
};

CopyShape copy_shape(int threads, int unroll, int64_t jobs, int64_t min_span_bytes, int programs) {
    int shift = 0;
    while ((1 << (shift + 1)) <= threads) ++shift;
    if (min_span_bytes > 0) {
        const int64_t vectors = min_span_bytes / 16;
        while (shift > 6 && (int64_t(1) << shift) * unroll > 2 * vectors) --shift;
    }
    const int64_t per_pass = threads >> shift;
    return CopyShape{shift, grid_for((jobs + per_pass - 1) / per_pass, programs)};
}

// The pieces kernels' grid: ceil(shortest span / 1 KiB) pieces per span (at
// most kMaxPieces; a longer span's last wave loops over the rest) times the
// spans in x, the blocks in y, at most kMaxPieceBlocks blocks a launch (the
// grid's y limit HIP states for every device).
constexpr int64_t kMaxPieces = 1024;
constexpr int64_t kMaxPieceWorkgroups = int64_t(1) << 25;
constexpr int64_t kMaxPieceBlocks = 65535;

int64_t span_pieces(int64_t min_span_bytes) {
    const int64_t pieces = (min_span_bytes + kPieceBytes - 1) / kPieceBytes;
    return pieces < 1 ? 1 : pieces > kMaxPieces ? kMaxPieces : pieces;
}

// Whether a copy launch goes by pieces: a grid sized to the work (programs <= 0), a known span length and
// a grid x dimension in range.
bool by_pieces(int64_t n_spans, int64_t min_span_bytes, int programs) {
    return programs <= 0 && min_span_bytes > 0 && n_spans * span_pieces(min_span_bytes) <= kMaxPieceWorkgroups;
}

template <bool kGather>
void launch_pieces(const int64_t* blocks, int64_t n_blocks, const int64_t* offs, const int64_t* bases,
                   const int64_t* pitches, const int64_t* words, int64_t n_spans, int64_t min_span_bytes,
                   char* records, int64_t record_pitch, hipStream_t stream) {
    const int64_t pieces = span_pieces(min_span_bytes);
    for (int64_t first = 0; first < n_blocks; first += kMaxPieceBlocks) {
        const int64_t count = n_blocks - first < kMaxPieceBlocks ? n_blocks - first : kMaxPieceBlocks;
        const dim3 grid(static_cast<unsigned>(n_spans * pieces), static_cast<unsigned>(count));
        hipLaunchKernelGGL(kGather ? gather_pieces_kernel : scatter_pieces_kernel, grid, dim3(64), 0, stream,
                           blocks + first, offs, bases, pitches, words, static_cast<uint32_t>(pieces),
                           records + first * record_pitch, record_pitch);
        check_launch(kGather ? "gather" : "scatter");
    }
}

struct CrcPlan {
    int groups;       // 4 KiB groups per stripe (one wave's job)
    int64_t stripes;  // per record, at most kCrcMaxStripes
    uint64_t pad;     // virtual zero bytes in front of each record
};

// Stripes of `groups` 1 KiB groups, the first one padded in front.  A stripe
// is one wave's job and costs its groups plus about two groups' worth of
// per-lane shifts and the wave's reduction; whole groups of padding cost
// nothing.  The resident waves (16 per CU) take about
// ceil(jobs / kCrcResidentWaves) rounds, so the plan picks the stripe count
// (at most kCrcMaxStripes, and at most max_partials / n_records when a
// workspace bounds it) that minimises rounds * (groups + 2): eight 288 KiB
// stripes per Qwen3-8B record of a 512-record session (4096 jobs, one round).
CrcPlan crc_plan(uint64_t record_bytes, int64_t n_records, int64_t max_partials = 0) {
    const uint64_t total = record_bytes ? (record_bytes + kCrcGroup - 1) / kCrcGroup : 1;
    const uint64_t n = n_records > 0 ? static_cast<uint64_t>(n_records) : 1;
    uint64_t cap = kCrcMaxStripes;
    if (max_partials > 0) cap = std::min<uint64_t>(cap, std::max<uint64_t>(1, static_cast<uint64_t>(max_partials) / n));
    cap = std::min<uint64_t>(cap, total);
    CrcPlan plan{static_cast<int>(total), 1, 0};
    uint64_t best = ~uint64_t(0);
    for (uint64_t s = 1; s <= cap; ++s) {
        const uint64_t g = (total + s - 1) / s;
        const uint64_t stripes = (total + g - 1) / g;
        const uint64_t rounds = (n * stripes + kCrcResidentWaves - 1) / kCrcResidentWaves;
        const uint64_t cost = rounds * (g + 2);
        if (cost < best) {
            best = cost;
            plan.groups = static_cast<int>(g);
            plan.stripes = static_cast<int64_t>(stripes);
        }
    }
    plan.pad = static_cast<uint64_t>(plan.stripes) * plan.groups * kCrcGroup - record_bytes;
    return plan;
}

// Largest grid of the CRC32C launch: two workgroups per CU.  The jobs are
// shared out statically over the waves, so a grid of the resident count
// leaves every wave one round of jobs.
constexpr unsigned kCrcGrid = 512;

// Whether a launch combines each record's stripes inside one workgroup
// (crc_records_kernel, one launch, no partials in memory): when a record's
// stripes fit the workgroup's 16 waves and the records still give the chip at
// least half its waves.
bool crc_in_group(const CrcPlan& plan, int64_t n_records) {
    return plan.stripes <= kCrcWaves && n_records * plan.stripes >= kCrcResidentWaves / 2;
}

// Queue the launches of out[i] = CRC32C of record i; `partial` (plan.stripes
// words per record) is used unless the stripes combine in their workgroup.
void launch_crc32c(const void* records, uint64_t record_bytes, uint64_t record_pitch, int64_t n_records,
                   uint32_t prior, uint32_t* out, uint32_t* partial, const CrcPlan& plan, hipStream_t s) {
    // The aligned kernels load 16-byte words at 32-bit record offsets, and a record of fewer than 16 bytes
    // has no word to stand in for a stripe's padding (crc_stripe_first).
    const bool aligned = (reinterpret_cast<uintptr_t>(records) % 16 == 0) && (record_pitch % 16 == 0) &&
                         (record_bytes % 16 == 0) && record_bytes >= 16 && record_bytes < (uint64_t(1) << 31);
    const int64_t jobs = n_records * plan.stripes;
    if (jobs > (int64_t(1) << 31)) throw std::runtime_error("CRC32C: too many records in one call");
    const auto* base = static_cast<const uint8_t*>(records);
    CrcStripePowers powers;
    const uint64_t stripe_bytes = static_cast<uint64_t>(plan.groups) * kCrcGroup;
    for (int i = 0; i < 6; ++i) powers.p[i] = host_xpow8n(stripe_bytes << i);
    const uint32_t init_term = host_shift(~prior, record_bytes);
    if (crc_in_group(plan, n_records)) {
        const int64_t per_group = kCrcWaves / plan.stripes;
        const unsigned grid = grid_for((n_records + per_group - 1) / per_group, kCrcGrid);
        const int stripes = static_cast<int>(plan.stripes);
        if (aligned)
            hipLaunchKernelGGL(crc_records_kernel<true>, dim3(grid), dim3(kCrcThreads), 0, s, base, record_pitch,
                               n_records, stripes, plan.groups, plan.pad, powers, init_term, out);
        else
            hipLaunchKernelGGL(crc_records_kernel<false>, dim3(grid), dim3(kCrcThreads), 0, s, base, record_pitch,
                               n_records, stripes, plan.groups, plan.pad, powers, init_term, out);
        check_launch("crc32c records");
        return;
    }
    if (!partial) throw std::runtime_error("CRC32C workspace missing");
    const unsigned grid = grid_for((jobs + kCrcWaves - 1) / kCrcWaves, kCrcGrid);
    if (aligned)
        hipLaunchKernelGGL(crc_stripes_kernel<true>, dim3(grid), dim3(kCrcThreads), 0, s, base, record_pitch,
                           n_records, plan.stripes, plan.groups, plan.pad, partial);
    else
        hipLaunchKernelGGL(crc_stripes_kernel<false>, dim3(grid), dim3(kCrcThreads), 0, s, base, record_pitch,
                           n_records, plan.stripes, plan.groups, plan.pad, partial);
    check_launch("crc32c stripes");
    hipLaunchKernelGGL(crc_combine_kernel, dim3(static_cast<unsigned>((n_records + 3) / 4)), dim3(256), 0, s, partial,
                       n_records, static_cast<int>(plan.stripes), powers, init_term, out);
    check_launch("crc32c combine");
}

// The no-allocation entry point's workspace: one array per device, holding
// the stripes' partial CRCs of one call.  Its address on each device is
// looked up once (hipGetSymbolAddress) with that device current.
constexpr int64_t kStaticCrcPartials = 65536;  // 256 KiB
constexpr int64_t kStaticCrcMaxRecords = kStaticCrcPartials;
__device__ __align__(256) uint32_t scratch[kStaticCrcPartials];
uint32_t* g_scratch_ptr[64];

// With `device` current: look up the array's address on it, once.
void init_static_crc_workspace(int device) {
    std::lock_guard<std::mutex> lock(g_table_mutex);
    if (g_scratch_ptr[device]) return;
    void* ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || !ptr)
        throw std::runtime_error(std::string("CRC32C static workspace address: ") + hipGetErrorString(rc));
    g_scratch_ptr[device] = static_cast<uint32_t*>(ptr);
}

// The current device's array and tables, set up by kvsnap_kernels_init: the
// no-allocation entry point makes no synchronous call of its own.
uint32_t* static_crc_workspace() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64)
        throw std::runtime_error("no current HIP device for the CRC32C workspace");
    std::lock_guard<std::mutex> lock(g_table_mutex);
    if (!g_scratch_ptr[device] || !g_tables_ready[device])
        throw std::runtime_error("CRC32C without allocation: call kvsnap_kernels_init for this device first");
    return g_scratch_ptr[device];
}

// CUs to themselves.  A gfx950 CU has 160 KiB of LDS.  The kernels that hold
// a few CUs for a long time -- the link-bound copies (a small grid whose waves
// wait on the host link: the restore, the checked restore from pinned memory,
// the gathers into pinned memory) and the SHA-256 chains (tens of ms) -- ask
// for every byte of LDS they do not use, so no other workgroup that uses LDS
// can share their CU.  Beside a copy wave a SHA-256 round wave slows (range
// launches took 2.5-3.5 ms beside the restore kernel, 1.8 ms alone); and an
// engine's workgroup placed beside a SHA-256 workgroup gets the VALU issue
// slots its round waves leave (they issue in about 84 % of them), so a
// decode step whose workgroups are dealt evenly over the chip waits for the
// ones on those CUs (the synthetic decode's median step went from 0.80 to
// 0.75 ms beside hashed saves once the SHA-256 workgroups took whole CUs).
// The cost is a few CUs (one per SHA-256 group of 64 records, one per copy
// workgroup) that the engine's LDS-using kernels leave alone.
constexpr unsigned kCuLds = 160 * 1024;
constexpr unsigned kCopyLdsFence = kCuLds;                                        // plain copies: no LDS of their own
constexpr unsigned kCheckedLdsFence = kCuLds - sizeof(uint32_t) * kCheckedLdsWords;  // the checked copies' tables
constexpr unsigned kShaLdsFence = kCuLds - sizeof(ShaSchedule);
static_assert(sizeof(ShaSchedule) < kCuLds, "a SHA-256 workgroup fits a CU");

}  // namespace

extern "C" {

int kvsnap_kernels_abi_version() { return 2; }

int kvsnap_kernels_init(int device) {
    return guard([&] {
        if (device < 0 || device >= 64) throw std::runtime_error("device index out of range");
        int previous = 0;
        hipError_t rc = hipGetDevice(&previous);
        if (rc != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(rc));
        rc = hipSetDevice(device);
        if (rc != hipSuccess) throw std::runtime_error(std::string("hipSetDevice: ") + hipGetErrorString(rc));
        try {
            ensure_crc_tables();
            init_static_crc_workspace(device);
        } catch (...) {
            (void)hipSetDevice(previous);
            throw;
        }
        rc = hipSetDevice(previous);
        if (rc != hipSuccess) throw std::runtime_error(std::string("hipSetDevice: ") + hipGetErrorString(rc));
    });
}

int kvsnap_restore_blocks(const int64_t* sources, const int64_t* blocks, int64_t n_blocks,
                          const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                          const int64_t* span_words, int64_t n_spans, int64_t min_span_bytes, int programs,
                          uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0 || n_spans < 0) throw std::runtime_error("negative restore size");
        if (n_blocks == 0 || n_spans == 0) return;
        if (!sources || !blocks || !span_offsets || !span_bases || !span_pitches || !span_words)
            throw std::runtime_error("restore tables must be device pointers");
        const CopyShape shape = copy_shape(kRestoreThreads, kRestoreUnroll, n_blocks * n_spans, min_span_bytes,
                                           programs);
        hipLaunchKernelGGL(restore_kernel, dim3(shape.grid), dim3(kRestoreThreads), kCopyLdsFence,
                           reinterpret_cast<hipStream_t>(stream), sources, blocks, n_blocks, span_offsets,
                           span_bases, span_pitches, span_words, n_spans, shape.lane_shift);
        check_launch("restore");
    });
}

int kvsnap_gather_blocks_checked(const int64_t* dests, const int64_t* blocks, int64_t n_blocks,
                                 const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                                 const int64_t* span_words, int64_t n_spans, void* stage, int64_t stage_pitch,
                                 int programs, uint32_t* partial, uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0 || n_spans < 0) throw std::runtime_error("negative gather size");
        if (n_blocks == 0 || n_spans == 0) return;
        if (!dests || !blocks || !span_offsets || !span_bases || !span_pitches || !span_words || !partial)
            throw std::runtime_error("checked gather tables and partials must be device pointers");
        if (reinterpret_cast<uintptr_t>(partial) % 4) throw std::runtime_error("checked gather partials misaligned");
        if (stage && (stage_pitch < 0 || reinterpret_cast<uintptr_t>(stage) % 8 || stage_pitch % 8))
            throw std::runtime_error("checked gather stage must be 8-byte aligned with a non-negative pitch");
        ensure_crc_tables();
        // A small grid (programs > 0) writes over the host link: 1024-lane workgroups on whole CUs (the LDS
        // fence).  A full grid is an HBM pass of 256-lane workgroups.
        const bool link = programs > 0;
        const int64_t waves = (link ? kGatherLinkThreads : kRestoreThreads) / 64;
        const unsigned grid = grid_for((n_blocks * n_spans + waves - 1) / waves, programs);
        const unsigned lds = link ? kCheckedLdsFence : 0;
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        char* stage_at = static_cast<char*>(stage);
        const int64_t pitch = stage ? stage_pitch : 0;
        if (link && stage)
            hipLaunchKernelGGL((gather_checked_kernel<true, kGatherLinkThreads>), dim3(grid), dim3(kGatherLinkThreads),
                               lds, s, dests, blocks, n_blocks, span_offsets, span_bases, span_pitches, span_words,
                               n_spans, stage_at, pitch, partial);
        else if (link)
            hipLaunchKernelGGL((gather_checked_kernel<false, kGatherLinkThreads>), dim3(grid),
                               dim3(kGatherLinkThreads), lds, s, dests, blocks, n_blocks, span_offsets, span_bases,
                               span_pitches, span_words, n_spans, stage_at, pitch, partial);
        else if (stage)
            hipLaunchKernelGGL((gather_checked_kernel<true, kRestoreThreads>), dim3(grid), dim3(kRestoreThreads), lds,
                               s, dests, blocks, n_blocks, span_offsets, span_bases, span_pitches, span_words, n_spans,
                               stage_at, pitch, partial);
        else
            hipLaunchKernelGGL((gather_checked_kernel<false, kRestoreThreads>), dim3(grid), dim3(kRestoreThreads),
                               lds, s, dests, blocks, n_blocks, span_offsets, span_bases, span_pitches, span_words,
                               n_spans, stage_at, pitch, partial);
        check_launch("checked gather");
    });
}

int kvsnap_gather_crc32c_fits(uint64_t record_bytes) {
    return record_bytes > 0 && record_bytes % kCrcGroup == 0 && record_bytes < (uint64_t(1) << 31) ? 1 : 0;
}

int kvsnap_gather_crc32c(const int64_t* blocks, int64_t n_blocks, const int64_t* group_bases,
                         const int64_t* group_pitches, uint64_t record_bytes, void* out, int64_t out_pitch,
                         uint32_t* crcs, uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0) throw std::runtime_error("negative gather size");
        if (n_blocks == 0) return;
        if (!kvsnap_gather_crc32c_fits(record_bytes))
            throw std::runtime_error("gather with CRC32C: records must be whole KiB, under 2 GiB");
        if (!blocks || !group_bases || !group_pitches || !out || !crcs)
            throw std::runtime_error("gather with CRC32C: tables, records and CRC32Cs must be device pointers");
        if (reinterpret_cast<uintptr_t>(out) % 16 || out_pitch % 16 || static_cast<uint64_t>(out_pitch) < record_bytes)
            throw std::runtime_error("gather with CRC32C: records must be 16-byte aligned and not overlap");
        if (reinterpret_cast<uintptr_t>(crcs) % 4) throw std::runtime_error("gather with CRC32C: CRC32Cs misaligned");
        ensure_crc_tables();
        // At most 16 stripes a record, so a workgroup's 16 waves hold whole records.
        const CrcPlan plan = crc_plan(record_bytes, n_blocks, int64_t(kCrcWaves) * n_blocks);
        const int stripes = static_cast<int>(plan.stripes);
        const int64_t per_group = kCrcWaves / stripes;
        CrcStripePowers powers;
        const uint64_t stripe_bytes = static_cast<uint64_t>(plan.groups) * kCrcGroup;
        for (int i = 0; i < 6; ++i) powers.p[i] = host_xpow8n(stripe_bytes << i);
        const unsigned grid = grid_for((n_blocks + per_group - 1) / per_group, kCrcGrid);
        hipLaunchKernelGGL(gather_crc_kernel, dim3(grid), dim3(kCrcThreads), 0, reinterpret_cast<hipStream_t>(stream),
                           blocks, n_blocks, group_bases, group_pitches, stripes, plan.groups,
                           static_cast<int>(plan.pad / kCrcGroup), powers, host_shift(~0u, record_bytes),
                           static_cast<char*>(out), out_pitch, crcs);
        check_launch("gather with CRC32C");
    });
}

int kvsnap_restore_blocks_checked(const int64_t* sources, const int64_t* blocks, int64_t n_blocks,
                                  const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                                  const int64_t* span_words, int64_t n_spans, int programs, uint32_t* partial,
                                  uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0 || n_spans < 0) throw std::runtime_error("negative restore size");
        if (n_blocks == 0 || n_spans == 0) return;
        if (!sources || !blocks || !span_offsets || !span_bases || !span_pitches || !span_words || !partial)
            throw std::runtime_error("checked restore tables and partials must be device pointers");
        if (reinterpret_cast<uintptr_t>(partial) % 4) throw std::runtime_error("checked restore partials misaligned");
        ensure_crc_tables();
        constexpr int64_t waves = kRestoreThreads / 64;
        const unsigned grid = grid_for((n_blocks * n_spans + waves - 1) / waves, programs);
        // From pinned memory (a small grid) the checked restore waits on the link and takes whole CUs; from
        // device staging (programs <= 0, a full grid) it is an HBM pass and shares them.
        hipLaunchKernelGGL(restore_checked_kernel, dim3(grid), dim3(kRestoreThreads),
                           programs > 0 ? kCheckedLdsFence : 0,
                           reinterpret_cast<hipStream_t>(stream), sources, blocks, n_blocks, span_offsets,
                           span_bases, span_pitches, span_words, n_spans, partial);
        check_launch("checked restore");
    });
}

int kvsnap_restore_checked_crc32c(const uint32_t* partial, int64_t n_blocks, const int64_t* span_offsets,
                                  const int64_t* span_words, int64_t n_spans, uint64_t record_bytes, uint32_t* out,
                                  uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0 || n_spans < 0) throw std::runtime_error("negative record count");
        if (n_blocks == 0) return;
        if (n_spans > kMaxCheckedSpans) throw std::runtime_error("too many spans for the checked restore");
        if (!out || (n_spans && (!partial || !span_offsets || !span_words)))
            throw std::runtime_error("checked restore CRC32C needs device pointers");
        if (record_bytes >= kCheckedMaxShift) throw std::runtime_error("record too long for the checked CRC32C");
        ensure_crc_tables();
        const size_t lds = static_cast<size_t>(n_spans > 0 ? n_spans : 1) * sizeof(uint32_t);
        const int64_t groups = (n_blocks + kFinishThreads / 64 - 1) / (kFinishThreads / 64);
        hipLaunchKernelGGL(restore_checked_finish_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(groups, 1024))),
                           dim3(kFinishThreads), lds, reinterpret_cast<hipStream_t>(stream), partial, n_blocks,
                           span_offsets, span_words, n_spans, record_bytes, host_shift(~0u, record_bytes), out);
        check_launch("checked restore CRC32C");
    });
}

int kvsnap_scatter_blocks(const void* records, int64_t record_pitch, const int64_t* blocks, int64_t n_blocks,
                          const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                          const int64_t* span_words, int64_t n_spans, int64_t min_span_bytes, int programs,
                          uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0 || n_spans < 0 || record_pitch < 0) throw std::runtime_error("negative scatter size");
        if (n_blocks == 0 || n_spans == 0) return;
        if (!records || !blocks || !span_offsets || !span_bases || !span_pitches || !span_words)
            throw std::runtime_error("scatter tables must be device pointers");
        if (by_pieces(n_spans, min_span_bytes, programs)) {
            launch_pieces<false>(blocks, n_blocks, span_offsets, span_bases, span_pitches, span_words, n_spans,
                                 min_span_bytes, const_cast<char*>(static_cast<const char*>(records)), record_pitch,
                                 reinterpret_cast<hipStream_t>(stream));
            return;
        }
        const CopyShape shape = copy_shape(kScatterThreads, kScatterUnroll, n_blocks * n_spans, min_span_bytes,
                                           programs);
        hipLaunchKernelGGL(scatter_kernel, dim3(shape.grid), dim3(kScatterThreads), 0,
                           reinterpret_cast<hipStream_t>(stream), static_cast<const char*>(records), record_pitch,
                           blocks, n_blocks, span_offsets, span_bases, span_pitches, span_words, n_spans,
                           shape.lane_shift);
        check_launch("scatter");
    });
}

int kvsnap_gather_blocks(const int64_t* blocks, int64_t n_blocks, const int64_t* span_offsets,
                         const int64_t* span_bases, const int64_t* span_pitches, const int64_t* span_words,
                         int64_t n_spans, int64_t min_span_bytes, void* records, int64_t record_pitch, int programs,
                         uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0 || n_spans < 0 || record_pitch < 0) throw std::runtime_error("negative gather size");
        if (n_blocks == 0 || n_spans == 0) return;
        if (!records || !blocks || !span_offsets || !span_bases || !span_pitches || !span_words)
            throw std::runtime_error("gather tables must be device pointers");
        if (by_pieces(n_spans, min_span_bytes, programs)) {
            launch_pieces<true>(blocks, n_blocks, span_offsets, span_bases, span_pitches, span_words, n_spans,
                                min_span_bytes, static_cast<char*>(records), record_pitch,
                                reinterpret_cast<hipStream_t>(stream));
            return;
        }
        const CopyShape shape = copy_shape(kGatherThreads, kGatherUnroll, n_blocks * n_spans, min_span_bytes,
                                           programs);
        hipLaunchKernelGGL(gather_kernel, dim3(shape.grid), dim3(kGatherThreads), 0,
                           reinterpret_cast<hipStream_t>(stream), blocks, n_blocks, span_offsets, span_bases,
                           span_pitches, span_words, n_spans, static_cast<char*>(records), record_pitch,
                           shape.lane_shift);
        check_launch("gather");
    });
}

int kvsnap_gather_to_records(const int64_t* dests, const int64_t* blocks, int64_t n_blocks,
                             const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                             const int64_t* span_words, int64_t n_spans, int64_t min_span_bytes, int programs,
                             uintptr_t stream) {
    return guard([&] {
        if (n_blocks < 0 || n_spans < 0) throw std::runtime_error("negative gather size");
        if (n_blocks == 0 || n_spans == 0) return;
        if (!dests || !blocks || !span_offsets || !span_bases || !span_pitches || !span_words)
            throw std::runtime_error("gather tables must be device pointers");
        const CopyShape shape = copy_shape(kRestoreThreads, kRestoreUnroll, n_blocks * n_spans, min_span_bytes,
                                           programs);
        hipLaunchKernelGGL(gather_to_kernel, dim3(shape.grid), dim3(kRestoreThreads), kCopyLdsFence,
                           reinterpret_cast<hipStream_t>(stream), dests, blocks, n_blocks, span_offsets, span_bases,
                           span_pitches, span_words, n_spans, shape.lane_shift);
        check_launch("gather to records");
    });
}

int kvsnap_synth_decode(const int64_t* span_bases, const int64_t* span_pitches, const int64_t* span_words,
                        int64_t n_spans, const int64_t* block_table, int64_t n_seqs, int64_t blocks_per_seq,
                        uint32_t* out, int programs, uintptr_t stream) {
    return guard([&] {
        if (n_spans < 0 || n_seqs < 0 || blocks_per_seq < 0) throw std::runtime_error("negative decode size");
        if (n_spans == 0 || n_seqs == 0) return;
        if (!span_bases || !span_pitches || !span_words || !block_table || !out)
            throw std::runtime_error("decode tables must be device pointers");
        hipLaunchKernelGGL(synth_decode_kernel, dim3(grid_for(n_seqs * n_spans, programs)), dim3(kThreads), 0,
                           reinterpret_cast<hipStream_t>(stream), span_bases, span_pitches, span_words, n_spans,
                           block_table, n_seqs, blocks_per_seq, out);
        check_launch("synthetic decode");
    });
}

int kvsnap_copy_to_device(void* dst, const void* src, size_t nbytes, uintptr_t stream) {
    return guard([&] {
        if (nbytes == 0) return;
        if (!dst || !src) throw std::runtime_error("copy needs a device destination and a pinned source");
        const hipError_t rc = hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice,
                                             reinterpret_cast<hipStream_t>(stream));
        if (rc != hipSuccess) throw std::runtime_error(std::string("copy to device: ") + hipGetErrorString(rc));
    });
}

int kvsnap_copy_to_host(void* dst, const void* src, size_t nbytes, uintptr_t stream) {
    return guard([&] {
        if (nbytes == 0) return;
        if (!dst || !src) throw std::runtime_error("copy needs a pinned destination and a device source");
        const hipError_t rc = hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost,
                                             reinterpret_cast<hipStream_t>(stream));
        if (rc != hipSuccess) throw std::runtime_error(std::string("copy to host: ") + hipGetErrorString(rc));
    });
}

int kvsnap_zero_regions(void* base, const int64_t* offsets, const int64_t* lengths, int64_t n, uintptr_t stream) {
    return guard([&] {
        if (n < 0) throw std::runtime_error("negative region count");
        if (n == 0) return;
        if (!base || !offsets || !lengths) throw std::runtime_error("zero regions need device pointers");
        hipLaunchKernelGGL(zero_kernel, dim3(grid_for(n, 1024)), dim3(kThreads), 0,
                           reinterpret_cast<hipStream_t>(stream), static_cast<char*>(base), offsets, lengths, n);
        check_launch("zero");
    });
}

int kvsnap_synth_fill(uint64_t seed, int kind, const int64_t* span_bases, const int64_t* span_pitches,
                      const int64_t* span_words, const float* span_inv_scales, int64_t n_spans, int64_t first_block,
                      int64_t n_blocks, uintptr_t stream) {
    return guard([&] {
        if (kind < 0 || kind > 2) throw std::runtime_error("unknown synthetic kind");
        if (n_spans < 0 || n_blocks < 0 || first_block < 0) throw std::runtime_error("negative synth size");
        if (n_spans == 0 || n_blocks == 0) return;
        hipLaunchKernelGGL(synth_kernel, dim3(grid_for(n_blocks * n_spans, 8192)), dim3(kThreads), 0,
                           reinterpret_cast<hipStream_t>(stream), seed, kind, span_bases, span_pitches, span_words,
                           span_inv_scales, n_spans, first_block, n_blocks);
        check_launch("synth");
    });
}

size_t kvsnap_crc32c_workspace_bytes(uint64_t record_bytes, int64_t n_records) {
    if (n_records <= 0) return 0;
    return static_cast<size_t>(crc_plan(record_bytes, n_records).stripes) * static_cast<size_t>(n_records) *
           sizeof(uint32_t);
}

int kvsnap_crc32c_records(const void* records, uint64_t record_bytes, uint64_t record_pitch, int64_t n_records,
                          uint32_t prior, uint32_t* out, void* workspace, size_t workspace_bytes, uintptr_t stream) {
    return guard([&] {
        if (n_records < 0) throw std::runtime_error("negative record count");
        if (n_records == 0) return;
        if (!out || (!records && record_bytes)) throw std::runtime_error("CRC32C needs device pointers");
        const CrcPlan plan = crc_plan(record_bytes, n_records);
        const size_t need = static_cast<size_t>(plan.stripes) * static_cast<size_t>(n_records) * sizeof(uint32_t);
        if (!workspace || workspace_bytes < need) throw std::runtime_error("CRC32C workspace too small");
        ensure_crc_tables();
        launch_crc32c(records, record_bytes, record_pitch, n_records, prior, out, static_cast<uint32_t*>(workspace),
                      plan, reinterpret_cast<hipStream_t>(stream));
    });
}

int kvsnap_crc32c_records_noalloc(const void* records, uint64_t record_bytes, uint64_t record_pitch,
                                 int64_t n_records, uint32_t prior, uint32_t* out, uintptr_t stream) {
    return guard([&] {
        if (n_records < 0) throw std::runtime_error("negative record count");
        if (n_records == 0) return;
        if (n_records > kStaticCrcMaxRecords)
            throw std::runtime_error("CRC32C without allocation: at most 65536 records per call");
        if (!out || (!records && record_bytes)) throw std::runtime_error("CRC32C needs device pointers");
        const CrcPlan plan = crc_plan(record_bytes, n_records, kStaticCrcPartials);
        if (plan.stripes * n_records > kStaticCrcPartials)
            throw std::runtime_error("CRC32C without allocation: the static workspace is too small");
        uint32_t* partials = static_crc_workspace();    // refuses a device kvsnap_kernels_init has not set up
        launch_crc32c(records, record_bytes, record_pitch, n_records, prior, out, partials, plan,
                      reinterpret_cast<hipStream_t>(stream));
    });
}

uint64_t kvsnap_sha256_blocks(uint64_t record_bytes) {
    const uint64_t whole = record_bytes / 64;
    return whole + (record_bytes - 64 * whole + 9 <= 64 ? 1 : 2);
}

}  // extern "C"

namespace {

// The checks every SHA-256 range passes before a launch.
void check_sha_range(const void* records, uint64_t record_bytes, int64_t n_records, uint64_t first_block,
                     uint64_t end_block, const uint32_t* state, const uint8_t* out) {
    if (n_records < 0) throw std::runtime_error("negative record count");
    const uint64_t nblocks = kvsnap_sha256_blocks(record_bytes);
    if (first_block >= end_block || end_block > nblocks) throw std::runtime_error("SHA-256 block range out of order");
    if (!records && record_bytes) throw std::runtime_error("SHA-256 needs device pointers");
    if (end_block == nblocks && !out) throw std::runtime_error("SHA-256 needs an output for the last blocks");
    if ((first_block > 0 || end_block < nblocks) && !state)
        throw std::runtime_error("SHA-256 over part of the chain needs a state buffer");
    if (reinterpret_cast<uintptr_t>(out) % 16 || reinterpret_cast<uintptr_t>(state) % 16)
        throw std::runtime_error("SHA-256 output and state must be 16-byte aligned");
}

}  // namespace

extern "C" {

int kvsnap_sha256_ranges(int count, const uint64_t* records, const uint64_t* record_bytes,
                         const uint64_t* record_pitches, const int64_t* n_records, const uint64_t* first_blocks,
                         const uint64_t* end_blocks, const uint64_t* states, const uint64_t* outs, uintptr_t stream) {
    return guard([&] {
        if (count < 0 || count > kShaMaxRanges) throw std::runtime_error("SHA-256: 0 to 8 ranges per launch");
        if (count && (!records || !record_bytes || !record_pitches || !n_records || !first_blocks || !end_blocks ||
                      !states || !outs))
            throw std::runtime_error("SHA-256 ranges need every table");
        ShaRanges ranges{};
        int used = 0;
        int64_t groups = 0;
        bool aligned = true;
        for (int i = 0; i < count; ++i) {
            const auto* base = reinterpret_cast<const uint8_t*>(records[i]);
            auto* state = reinterpret_cast<uint32_t*>(states[i]);
            auto* out = reinterpret_cast<uint8_t*>(outs[i]);
            check_sha_range(base, record_bytes[i], n_records[i], first_blocks[i], end_blocks[i], state, out);
            if (n_records[i] == 0) continue;
            aligned = aligned && records[i] % 16 == 0 && record_pitches[i] % 16 == 0;
            ranges.r[used++] = ShaRange{base, record_bytes[i], record_pitches[i], n_records[i], first_blocks[i],
                                        end_blocks[i], state, reinterpret_cast<uint32_t*>(out)};
            groups = std::max<int64_t>(groups, (n_records[i] + kShaRecords - 1) / kShaRecords);
        }
        if (!used) return;
        if (groups > (int64_t(1) << 30)) throw std::runtime_error("SHA-256: too many records");
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>(used));
        if (aligned)
            hipLaunchKernelGGL(sha256_ranges_kernel<true>, grid, dim3(kShaThreads), kShaLdsFence, s, ranges);
        else
            hipLaunchKernelGGL(sha256_ranges_kernel<false>, grid, dim3(kShaThreads), kShaLdsFence, s, ranges);
        check_launch("sha256 ranges");
    });
}

int kvsnap_sha256_records_range(const void* records, uint64_t record_bytes, uint64_t record_pitch,
                                int64_t n_records, uint64_t first_block, uint64_t end_block, uint32_t* state,
                                uint8_t* out, uintptr_t stream) {
    return guard([&] {
        if (n_records < 0) throw std::runtime_error("negative record count");
        if (n_records == 0) return;
        check_sha_range(records, record_bytes, n_records, first_block, end_block, state, out);
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        const bool aligned = (reinterpret_cast<uintptr_t>(records) % 16 == 0) && (record_pitch % 16 == 0);
        const unsigned grid = static_cast<unsigned>((n_records + kShaRecords - 1) / kShaRecords);
        const auto* base = static_cast<const uint8_t*>(records);
        auto* words = reinterpret_cast<uint32_t*>(out);
        if (aligned)
            hipLaunchKernelGGL(sha256_kernel<true>, dim3(grid), dim3(kShaThreads), kShaLdsFence, s, base, record_bytes,
                               record_pitch, n_records, first_block, end_block, state, words);
        else
            hipLaunchKernelGGL(sha256_kernel<false>, dim3(grid), dim3(kShaThreads), kShaLdsFence, s, base, record_bytes,
                               record_pitch, n_records, first_block, end_block, state, words);
        check_launch("sha256");
    });
}

int kvsnap_sha256_records(const void* records, uint64_t record_bytes, uint64_t record_pitch, int64_t n_records,
                          uint8_t* out, uintptr_t stream) {
    return kvsnap_sha256_records_range(records, record_bytes, record_pitch, n_records, 0,
                                       kvsnap_sha256_blocks(record_bytes), nullptr, out, stream);
}

int kvsnap_sha_round_probe(uint32_t seed, int reps, uint64_t* out, uintptr_t stream) {
    return guard([&] {
        if (reps < kShaProbeUnroll || reps % kShaProbeUnroll || reps > (1 << 24))
            throw std::runtime_error("SHA-256 round probe: reps a multiple of 16, at most 2^24");
        if (!out || reinterpret_cast<uintptr_t>(out) % 8) throw std::runtime_error("SHA-256 round probe: bad output");
        hipLaunchKernelGGL(sha_round_probe_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), seed,
                           reps, out);
        check_launch("SHA-256 round probe");
    });
}

int kvsnap_read_probe(const void* src, uint64_t bytes, uint32_t* sink, uintptr_t stream) {
    return guard([&] {
        if (!src || reinterpret_cast<uintptr_t>(src) % 16 || bytes == 0 || bytes % 16)
            throw std::runtime_error("read probe: a 16-byte aligned buffer of a positive multiple of 16 bytes");
        if (!sink || reinterpret_cast<uintptr_t>(sink) % 4) throw std::runtime_error("read probe: bad sink");
        hipLaunchKernelGGL(read_probe_kernel, dim3(kReadProbeGroups), dim3(kReadProbeLanes), 0,
                           reinterpret_cast<hipStream_t>(stream), static_cast<const u32x4*>(src), bytes / 16, sink);
        check_launch("read probe");
    });
}

int kvsnap_copy_probe(const void* src, void* dst, uint64_t bytes, uintptr_t stream) {
    return guard([&] {
        if (!src || !dst || (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 || bytes == 0 ||
            bytes % 16 || bytes > (uint64_t{1} << 40))
            throw std::runtime_error("copy probe: 16-byte aligned buffers of a positive multiple of 16 bytes, at most 1 TiB");
        const uint64_t words = bytes / 16;
        hipLaunchKernelGGL(copy_probe_kernel, dim3(static_cast<uint32_t>((words + 63) / 64)), dim3(64), 0,
                           reinterpret_cast<hipStream_t>(stream), static_cast<const u32x4*>(src),
                           static_cast<u32x4*>(dst), words);
        check_launch("copy probe");
    });
}

int kvsnap_stream_create(int device, uintptr_t* stream) {
    return guard([&] {
        if (!stream) throw std::runtime_error("stream create needs an output");
        int current = 0;
        if (hipGetDevice(&current) != hipSuccess) throw std::runtime_error("stream create: no current device");
        if (hipSetDevice(device) != hipSuccess) throw std::runtime_error("stream create: bad device");
        hipStream_t s = nullptr;
        const hipError_t rc = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        const hipError_t back = hipSetDevice(current);
        if (rc != hipSuccess) throw std::runtime_error(std::string("stream create: ") + hipGetErrorString(rc));
        if (back != hipSuccess) {
            (void)hipStreamDestroy(s);
            throw std::runtime_error("stream create: could not restore the current device");
        }
        *stream = reinterpret_cast<uintptr_t>(s);
    });
}

int kvsnap_stream_destroy(uintptr_t stream) {
    return guard([&] {
        if (!stream) return;
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        hipError_t rc = hipStreamSynchronize(s);
        if (rc == hipSuccess) rc = hipStreamDestroy(s);
        if (rc != hipSuccess) throw std::runtime_error(std::string("stream destroy: ") + hipGetErrorString(rc));
    });
}

int kvsnap_hold_stream(uintptr_t stream, int iters) {
    return guard([&] {
        if (iters < 0 || iters > kMaxHoldIters) throw std::runtime_error("hold length out of range");
        hipLaunchKernelGGL(hold_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), iters);
        check_launch("hold");
    });
}

}  // extern "C"
