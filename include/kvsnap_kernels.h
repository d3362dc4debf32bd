/*
 * gfx950 kernels of the snapshot dataplane, built into
 * kvsnap_amd/_native/libkvsnap_hip.so.
 *
 * Tables and buffers are device addresses (hipMalloc'd or torch tensors;
 * `sources` may also be pinned host addresses from the pool, which the restore
 * kernel reads in place over the host link).  Every entry point launches on
 * `stream` (a hipStream_t as an integer), returns 0 once the launch is queued
 * and -1 with kvsnap_cuda_error() set if the arguments are refused or the
 * launch fails.  Nothing is allocated.
 *
 * Span tables: span s of block b lives at span_bases[s] + b * span_pitches[s]
 * (bytes), is span_words[s] 8-byte words long, and sits at byte
 * span_offsets[s] of the block's packed record.  One span per layer for the
 * reference's [blocks, H, N, C] caches (in sorted layer-name order), two per
 * layer (K, then V) for [2, blocks, N, H, C] caches.
 *
 * Copy launches take `min_span_bytes`, the length of the shortest span (0 if
 * unknown): a launch-shape hint that never changes what is copied.
 * `programs` caps the grid (<= 0: as many workgroups as the work needs).  A
 * gather or scatter with programs <= 0 and a known hint goes one 64-lane
 * workgroup per KiB of a span; otherwise a workgroup takes (block, span)
 * jobs in turn, and short spans (a tensor-parallel rank's shard, fp8 caches)
 * are copied several to a workgroup.
 */
#ifndef KVSNAP_KERNELS_H
#define KVSNAP_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Always 2 (2 added min_span_bytes to the copy launches). */
int kvsnap_kernels_abi_version(void);

/* Set-up for `device`, synchronous: uploads the CRC32C tables and looks up the
 * no-allocation entry point's static array on that device (the current device
 * is restored on return).  Idempotent.  The other entry points set up a
 * device on their first call there; kvsnap_crc32c_records_noalloc refuses a
 * device that this call has not set up.  No counterpart in the reference
 * (its copy kernel needs no tables); TorchBlockDataPlane.warm_up calls it. */
int kvsnap_kernels_init(int device);

/* Restore: for every (block i, span s), copy span_words[s] words from
 * sources[i] + span_offsets[s] to span_bases[s] + blocks[i] * span_pitches[s].
 * Replaces the Triton launch copy_host_blocks(sources, blocks,
 * layer_offsets, layer_bases, layer_pitches, layer_words),
 * kvsnap/connector/copy_kernel.py:43-49 (kernel :22-40), called from
 * kvsnap/connector/dataplane.py:374. */
int kvsnap_restore_blocks(const int64_t* sources, const int64_t* blocks, int64_t n_blocks,
                          const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                          const int64_t* span_words, int64_t n_spans, int64_t min_span_bytes, int programs,
                          uintptr_t stream);

/* The save's gather with every record's CRC32C folded in (the checked
 * restore's inverse): for every (block i, span s), copy span_words[s] words
 * from span_bases[s] + blocks[i] * span_pitches[s] to dests[i] +
 * span_offsets[s] (pinned host memory or device memory) and, when `stage` is
 * not NULL, also to stage + i * stage_pitch + span_offsets[s] (device
 * memory), and leave the span's raw CRC in partial[i * n_spans + s] for
 * kvsnap_restore_checked_crc32c.  One wave per (block, span); `programs`
 * caps the grid (<= 0: one workgroup per four jobs).  Replaces save_gather's
 * index_select + cat and D2H (kvsnap/connector/dataplane.py:409-427) followed
 * by the per-block host CRC32C (kvsnap/connector/volatile.py:151,
 * kvsnap/store/store.py:622) for saves whose records are written straight
 * into pinned memory. */
int kvsnap_gather_blocks_checked(const int64_t* dests, const int64_t* blocks, int64_t n_blocks,
                                 const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                                 const int64_t* span_words, int64_t n_spans, void* stage, int64_t stage_pitch,
                                 int programs, uint32_t* partial, uintptr_t stream);

/* Whether kvsnap_gather_crc32c takes records of record_bytes: 1 for whole
 * KiB under 2 GiB, else 0. */
int kvsnap_gather_crc32c_fits(uint64_t record_bytes);

/* The save's gather into device records with every record's CRC32C, in one
 * HBM pass: record i (block blocks[i]) to out + i * out_pitch, its CRC32C
 * (init/xorout ~0) to crcs[i].  For layouts whose spans are whole KiB: the
 * record's 1 KiB group g comes from group_bases[g] + blocks[i] *
 * group_pitches[g] (16-byte aligned; record_bytes / 1024 groups, built once
 * per layout from the span table).  out and out_pitch 16-byte aligned.
 * Replaces save_gather's index_select + cat into device staging
 * (kvsnap/connector/dataplane.py:409-417) together with the per-block
 * CRC32C of each record (kvsnap/connector/volatile.py:151,
 * kvsnap/store/store.py:622), which otherwise reads the staged records
 * again. */
int kvsnap_gather_crc32c(const int64_t* blocks, int64_t n_blocks, const int64_t* group_bases,
                         const int64_t* group_pitches, uint64_t record_bytes, void* out, int64_t out_pitch,
                         uint32_t* crcs, uintptr_t stream);

/* Checked restore: the copy of kvsnap_restore_blocks (any span length and
 * 8-byte alignment), and partial[i * n_spans + s] = the raw CRC32C (zero
 * initial value, no final xor) of block i's span s at the span's end, folded
 * from the bytes as they are copied.  kvsnap_restore_checked_crc32c then
 * gives each block's CRC32C from its partials.  Replaces the host
 * CRC32C checks that precede a restore from pinned memory:
 * VolatileOwner.borrow(verify_checksums=True), kvsnap/connector/volatile.py:
 * 302-305, and the staged fetch's check at kvsnap/connector/vllm.py:531
 * (kvsnap_crc32c_extend, csrc/dataplane/io.cpp:39-44), each of which reads
 * the block once more on the host before the copy. */
int kvsnap_restore_blocks_checked(const int64_t* sources, const int64_t* blocks, int64_t n_blocks,
                                  const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                                  const int64_t* span_words, int64_t n_spans, int programs, uint32_t* partial,
                                  uintptr_t stream);

/* out[i] = CRC32C (init/xorout ~0) of the record_bytes of block i whose spans
 * (span_offsets / span_words, the restore's tables; at most 8192 spans) tile
 * the record, from the n_blocks * n_spans partials kvsnap_restore_blocks_checked
 * wrote.  Bit-exact with kvsnap_crc32c_extend(record, record_bytes, 0). */
int kvsnap_restore_checked_crc32c(const uint32_t* partial, int64_t n_blocks, const int64_t* span_offsets,
                                  const int64_t* span_words, int64_t n_spans, uint64_t record_bytes, uint32_t* out,
                                  uintptr_t stream);

/* Gather: block blocks[i]'s spans packed into records + i * record_pitch.
 * Replaces save_gather's torch.cat([raw.index_select(0, ids) ...], out=stage),
 * kvsnap/connector/dataplane.py:416-417. */
int kvsnap_gather_blocks(const int64_t* blocks, int64_t n_blocks, const int64_t* span_offsets,
                         const int64_t* span_bases, const int64_t* span_pitches, const int64_t* span_words,
                         int64_t n_spans, int64_t min_span_bytes, void* records, int64_t record_pitch, int programs,
                         uintptr_t stream);

/* Gather into per-block destinations: block blocks[i]'s spans written to
 * dests[i] + span_offsets[s], typically pinned host records written in place
 * over the host link (a save without a device staging buffer).  Replaces the
 * same gather (kvsnap/connector/dataplane.py:416-417) followed by its D2H
 * copies into per-block allocations (:418-427). */
int kvsnap_gather_to_records(const int64_t* dests, const int64_t* blocks, int64_t n_blocks,
                             const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                             const int64_t* span_words, int64_t n_spans, int64_t min_span_bytes, int programs,
                             uintptr_t stream);

/* Scatter: the record at records + i * record_pitch, in device memory, into
 * block blocks[i]'s spans; the gather's inverse.  The last step of a restore
 * whose records were first staged and CRC-checked on the device: replaces the
 * reference's restore launch (kvsnap/connector/copy_kernel.py:43-49) for
 * device-resident sources, with an HBM-to-HBM grid shape. */
int kvsnap_scatter_blocks(const void* records, int64_t record_pitch, const int64_t* blocks, int64_t n_blocks,
                          const int64_t* span_offsets, const int64_t* span_bases, const int64_t* span_pitches,
                          const int64_t* span_words, int64_t n_spans, int64_t min_span_bytes, int programs,
                          uintptr_t stream);

/* Copy nbytes from pinned host memory to device memory on `stream` (the DMA
 * engines, hipMemcpyAsync).  The restore's "dma" mode stages records with it
 * and then scatters them with kvsnap_scatter_blocks, so that a restore's
 * host-to-device traffic runs on the copy engines beside a save's
 * device-to-host copies; the reference has no counterpart (its restore reads
 * pinned memory in place, kvsnap/connector/copy_kernel.py:22-40). */
int kvsnap_copy_to_device(void* dst, const void* src, size_t nbytes, uintptr_t stream);

/* Copy nbytes from device memory to pinned host memory on `stream` (the DMA
 * engines, hipMemcpyAsync); no reference counterpart.  With
 * kvsnap_copy_to_device, the plane times which copy engine a new restore
 * stream took (the pool's own device-to-host copies are kvsnap_pool_copy). */
int kvsnap_copy_to_host(void* dst, const void* src, size_t nbytes, uintptr_t stream);

/* Zero n byte ranges [base + offsets[i], + lengths[i]): the token slots past
 * the last computed token of a record.  Replaces the host memsets of
 * TorchBlockDataPlane._zero_tail, kvsnap/connector/dataplane.py:262-272. */
int kvsnap_zero_regions(void* base, const int64_t* offsets, const int64_t* lengths, int64_t n, uintptr_t stream);

/* Device bytes of scratch that kvsnap_crc32c_records needs for n records. */
size_t kvsnap_crc32c_workspace_bytes(uint64_t record_bytes, int64_t n_records);

/* out[i] = CRC32C (Castagnoli, reflected, init/xorout ~0, extending `prior`)
 * of the record_bytes at records + i * record_pitch.  Bit-exact with
 * kvsnap_crc32c_extend (csrc/dataplane/io.cpp:39-44); replaces its per-block
 * host calls at kvsnap/connector/volatile.py:151, kvsnap/store/store.py:622
 * and :717. */
int kvsnap_crc32c_records(const void* records, uint64_t record_bytes, uint64_t record_pitch, int64_t n_records,
                          uint32_t prior, uint32_t* out, void* workspace, size_t workspace_bytes, uintptr_t stream);

/* The CRC32C of kvsnap_crc32c_records with no allocation at all: no workspace
 * argument, and no hipMalloc, hipFree or allocating library call.  No
 * counterpart in the reference; for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid it).  When a
 * record's stripes do not combine inside their workgroup (few records), their
 * partial CRCs go to one static device array of 65536 words (256 KiB) per
 * GPU, held until the process ends: at most 65536 records per call (a larger
 * batch fails with an error before anything is queued).  Calls that overlap
 * on one GPU race on that array, so callers order them (one stream, or
 * events).  The array keeps the last call's partials; a call reads only what
 * it has written.  Call kvsnap_kernels_init(device) once first (it uploads
 * the tables and finds the array, synchronously): this entry point makes no
 * synchronous call, and refuses a device that was not set up. */
int kvsnap_crc32c_records_noalloc(const void* records, uint64_t record_bytes, uint64_t record_pitch,
                                  int64_t n_records, uint32_t prior, uint32_t* out, uintptr_t stream);

/* out[32 * i .. 32 * i + 31] = SHA-256 digest of record i (16-byte aligned
 * `out`).  Replaces hashlib.sha256(record) at kvsnap/connector/volatile.py:151
 * and kvsnap/store/store.py:622 (the blob id, blobs.py:33-36). */
int kvsnap_sha256_records(const void* records, uint64_t record_bytes, uint64_t record_pitch, int64_t n_records,
                          uint8_t* out, uintptr_t stream);

/* 64-byte compressions in one record's SHA-256 chain, padding included. */
uint64_t kvsnap_sha256_blocks(uint64_t record_bytes);

/* Compressions [first_block, end_block) of every record's SHA-256 chain:
 * from the initial value when first_block = 0, else from `state` (8 uint32
 * per record, left there by the previous range); the digest into `out` when
 * end_block = kvsnap_sha256_blocks(record_bytes), else the chaining state
 * back into `state`.  A series of ranges equals one kvsnap_sha256_records
 * call; each launch is short, so the stream's hardware queue (which other
 * streams of the process may share) is never held for a whole chain. */
int kvsnap_sha256_records_range(const void* records, uint64_t record_bytes, uint64_t record_pitch,
                                int64_t n_records, uint64_t first_block, uint64_t end_block, uint32_t* state,
                                uint8_t* out, uintptr_t stream);

/* Up to 8 independent kvsnap_sha256_records_range calls in one launch (no
 * reference counterpart: the reference hashes each save's blocks on host
 * threads).  Range i is the i-th entry of every host array: records address,
 * record bytes and pitch, record count, first and end block, state and out
 * addresses, each checked as kvsnap_sha256_records_range checks them.  Saves
 * hashing at the same time share each launch, so they hash side by side on
 * one stream instead of in turn. */
int kvsnap_sha256_ranges(int count, const uint64_t* records, const uint64_t* record_bytes,
                         const uint64_t* record_pitches, const int64_t* n_records, const uint64_t* first_blocks,
                         const uint64_t* end_blocks, const uint64_t* states, const uint64_t* outs, uintptr_t stream);

/* The SHA-256 round's own issue rate, measured on the GPU: one wave runs
 * `reps` (a multiple of 16) slots of sha256_kernel's round sequence with no
 * memory traffic, and out (3 device words) receives the shader-clock cycles,
 * the 100 MHz constant-clock ticks and a checksum.  No reference
 * counterpart: the bench's SHA-256 bound is priced from it. */
int kvsnap_sha_round_probe(uint32_t seed, int reps, uint64_t* out, uintptr_t stream);

/* The chip's read rate for a buffer of a given size, measured: one launch of
 * 256 workgroups of 1024 lanes (the CRC32C kernels' shape, one a CU) reads
 * the `bytes` (a positive multiple of 16, src 16-byte aligned) at `src` with
 * nontemporal 16-byte loads and does nothing else with them.  sink (4096
 * device words) receives one word a wave; their XOR is the XOR of the
 * buffer's 32-bit words.  No reference counterpart: the bench prices the
 * CRC32C kernels against it at the same size. */
int kvsnap_read_probe(const void* src, uint64_t bytes, uint32_t* sink, uintptr_t stream);

/* The chip's rate for a contiguous device-to-device copy of a given size,
 * measured: `bytes` (a positive multiple of 16, at most 1 TiB; src and dst
 * 16-byte aligned, not overlapping) copied with the gather and scatter
 * kernels' shape, one 64-lane workgroup a KiB and one nontemporal 16-byte
 * load and store a lane.  No reference counterpart: the bench prices the
 * gather and scatter kernels against it at the same size. */
int kvsnap_copy_probe(const void* src, void* dst, uint64_t bytes, uintptr_t stream);

/* Streams of the data plane's own (no reference counterpart; the reference
 * copies on one stream).  kvsnap_stream_create makes a non-blocking stream of
 * default priority on `device`; kvsnap_stream_destroy waits for its work and
 * frees it.  kvsnap_hold_stream queues one wave that sleeps `iters` rounds of
 * about 3.4 us (0 <= iters <= 30000) and ends: work queued on streams that
 * share the held stream's hardware queue waits behind it, which is how the
 * plane keeps its copy, restore and hash streams on queues of their own. */
int kvsnap_stream_create(int device, uintptr_t* stream);
int kvsnap_stream_destroy(uintptr_t stream);
int kvsnap_hold_stream(uintptr_t stream, int iters);

/* Seeded synthetic KV for benchmarks and tests (no reference counterpart):
 * every span of blocks [first_block, first_block + n_blocks) filled from a
 * counter-based generator keyed (seed, span, block, element); kind 0 bf16
 * ~N(0,1), 1 fp8-e4m3 of N(0,1) * span_inv_scales[s], 2 raw bytes. */
int kvsnap_synth_fill(uint64_t seed, int kind, const int64_t* span_bases, const int64_t* span_pitches,
                      const int64_t* span_words, const float* span_inv_scales, int64_t n_spans, int64_t first_block,
                      int64_t n_blocks, uintptr_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KVSNAP_KERNELS_H */
