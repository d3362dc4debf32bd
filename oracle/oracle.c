/*
 * CPU oracle for the KV snapshot dataplane -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's byte path, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, to check results.
 * Nothing in kvsnap_amd/ may link, load or call it.
 *
 * Each function names the reference file:line it restates (paths relative to
 * the simon-jd/kvsnap tree).  How each one is pinned (golden vectors, the
 * compiled reference io.cpp, library routines, closed forms) is listed in
 * oracle/__init__.py's header.
 */
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#if defined(__x86_64__)
#include <immintrin.h>
#include <nmmintrin.h>
#endif

/* ------------------------------------------------------------------------ */
/* CRC32C (Castagnoli, reflected polynomial 0x82F63B78, init/xorout ~0).     */
/* ------------------------------------------------------------------------ */

/* Bit-at-a-time textbook form; csrc/dataplane/io.cpp:16-25. */
uint32_t oracle_crc32c_bitwise(const void *data, size_t size, uint32_t prior)
{
    const uint8_t *p = (const uint8_t *)data;
    uint32_t state = ~prior;
    for (size_t i = 0; i < size; ++i) {
        state ^= p[i];
        for (int bit = 0; bit < 8; ++bit)
            state = (state >> 1) ^ (0x82F63B78u & (0u - (state & 1u)));
    }
    return ~state;
}

#if defined(__x86_64__)
/* SSE4.2 crc32 instruction, 8 bytes per step, then bytes; io.cpp:26-37. */
__attribute__((target("sse4.2")))
static uint32_t crc32c_hw(const void *data, size_t size, uint32_t prior)
{
    const uint8_t *p = (const uint8_t *)data;
    uint64_t state = (uint32_t)~prior;
    for (; size >= 8; size -= 8, p += 8) {
        uint64_t word;
        memcpy(&word, p, 8);
        state = _mm_crc32_u64(state, word);
    }
    uint32_t s32 = (uint32_t)state;
    for (; size; --size, ++p)
        s32 = _mm_crc32_u8(s32, *p);
    return ~s32;
}
#endif

/* Runtime dispatch as kvsnap_crc32c_extend does; io.cpp:39-44. */
uint32_t oracle_crc32c(const void *data, size_t size, uint32_t prior)
{
#if defined(__x86_64__)
    if (__builtin_cpu_supports("sse4.2"))
        return crc32c_hw(data, size, prior);
#endif
    return oracle_crc32c_bitwise(data, size, prior);
}

/* ------------------------------------------------------------------------ */
/* SHA-256, FIPS 180-4 section 6.2 (hashlib.sha256 at the reference's call   */
/* sites kvsnap/connector/volatile.py:151 and kvsnap/store/store.py:622).    */
/* ------------------------------------------------------------------------ */

static const uint32_t SHA_K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2,
};

static inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha_compress(uint32_t h[8], const uint8_t block[64])
{
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
        w[t] = (uint32_t)block[4 * t] << 24 | (uint32_t)block[4 * t + 1] << 16 |
               (uint32_t)block[4 * t + 2] << 8 | (uint32_t)block[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
        uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
        uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int t = 0; t < 64; ++t) {
        uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + SHA_K[t] + w[t];
        uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}

#if defined(__x86_64__)
/* The same compression with the x86 SHA extensions (Intel's published
 * SHA-NI method): state kept as ABEF/CDGH lane pairs, 4 rounds per
 * sha256rnds2 pair, message schedule by sha256msg1/msg2.  Used for the CPU
 * baseline; checked against sha_compress and hashlib. */
__attribute__((target("sha,sse4.1,ssse3")))
static void sha_compress_ni(uint32_t h[8], const uint8_t *p, size_t blocks)
{
    const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bLL, 0x0405060700010203LL);
    __m128i tmp = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i *)&h[0]), 0xB1);
    __m128i st1 = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i *)&h[4]), 0x1B);
    __m128i st0 = _mm_alignr_epi8(tmp, st1, 8);
    st1 = _mm_blend_epi16(st1, tmp, 0xF0);
    for (; blocks; --blocks, p += 64) {
        const __m128i save0 = st0, save1 = st1;
        __m128i m[4];
        for (int i = 0; i < 4; ++i)
            m[i] = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i *)(p + 16 * i)), bswap);
        for (int i = 0; i < 16; ++i) {
            __m128i wk = _mm_add_epi32(m[i & 3], _mm_loadu_si128((const __m128i *)&SHA_K[4 * i]));
            st1 = _mm_sha256rnds2_epu32(st1, st0, wk);
            if (i < 12) {
                __m128i next = _mm_sha256msg1_epu32(m[i & 3], m[(i + 1) & 3]);
                next = _mm_add_epi32(next, _mm_alignr_epi8(m[(i + 3) & 3], m[(i + 2) & 3], 4));
                m[i & 3] = _mm_sha256msg2_epu32(next, m[(i + 3) & 3]);
            }
            st0 = _mm_sha256rnds2_epu32(st0, st1, _mm_shuffle_epi32(wk, 0x0E));
        }
        st0 = _mm_add_epi32(st0, save0);
        st1 = _mm_add_epi32(st1, save1);
    }
    tmp = _mm_shuffle_epi32(st0, 0x1B);
    st1 = _mm_shuffle_epi32(st1, 0xB1);
    _mm_storeu_si128((__m128i *)&h[0], _mm_blend_epi16(tmp, st1, 0xF0));
    _mm_storeu_si128((__m128i *)&h[4], _mm_alignr_epi8(st1, tmp, 8));
}
#endif

static int use_sha_ni = -1;

/* 0: portable rounds only; 1: SHA extensions when the CPU has them. */
void oracle_sha256_select(int allow_extensions) { use_sha_ni = allow_extensions ? -1 : 0; }

static void sha_blocks(uint32_t h[8], const uint8_t *p, size_t blocks)
{
#if defined(__x86_64__)
    if (use_sha_ni < 0)
        use_sha_ni = __builtin_cpu_supports("sha") && __builtin_cpu_supports("sse4.1") ? 1 : 0;
    if (use_sha_ni) {
        sha_compress_ni(h, p, blocks);
        return;
    }
#endif
    for (size_t i = 0; i < blocks; ++i)
        sha_compress(h, p + 64 * i);
}

void oracle_sha256(const void *data, size_t size, uint8_t out[32])
{
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    const uint8_t *p = (const uint8_t *)data;
    size_t whole = size / 64;
    sha_blocks(h, p, whole);
    uint8_t tail[128];
    size_t rest = size - 64 * whole;
    memset(tail, 0, sizeof tail);
    memcpy(tail, p + 64 * whole, rest);
    tail[rest] = 0x80;
    size_t blocks = rest + 1 + 8 <= 64 ? 1 : 2;
    uint64_t bits = (uint64_t)size * 8u;
    for (int i = 0; i < 8; ++i)
        tail[64 * blocks - 1 - i] = (uint8_t)(bits >> (8 * i));
    sha_blocks(h, tail, blocks);
    for (int i = 0; i < 8; ++i) {
        out[4 * i] = (uint8_t)(h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(h[i] >> 8);
        out[4 * i + 3] = (uint8_t)h[i];
    }
}

/* ------------------------------------------------------------------------ */
/* Record geometry: gather, scatter, tail zeroing.                            */
/* A span s of block b lives at span_base[s] + b * span_pitch[s] and occupies */
/* record bytes [span_offset[s], span_offset[s] + span_bytes[s]).  For the   */
/* reference layout there is one span per layer, in sorted layer-name order  */
/* (kvsnap/connector/dataplane.py:226, 245-248, 283-317).                    */
/* ------------------------------------------------------------------------ */

/* save_gather's bytes: record i = concat over spans of block ids[i]'s span,
 * kvsnap/connector/dataplane.py:409-417 (index_select + cat, block-major). */
void oracle_gather(size_t n_spans, const uint64_t *span_base, const int64_t *span_pitch,
                   const int64_t *span_offset, const int64_t *span_bytes,
                   const int64_t *block_ids, size_t n_blocks, uint8_t *records, size_t block_bytes)
{
    for (size_t i = 0; i < n_blocks; ++i)
        for (size_t s = 0; s < n_spans; ++s)
            memcpy(records + i * block_bytes + span_offset[s],
                   (const uint8_t *)(uintptr_t)(span_base[s] + (uint64_t)(block_ids[i] * span_pitch[s])),
                   (size_t)span_bytes[s]);
}

/* The restore kernel's semantics: job (block i, span s) copies
 * span_bytes[s] from sources[i] + span_offset[s] to
 * span_base[s] + ids[i] * span_pitch[s]
 * (kvsnap/connector/copy_kernel.py:25-40; test_scatter_gather.py:71-76). */
void oracle_scatter(size_t n_spans, const uint64_t *span_base, const int64_t *span_pitch,
                    const int64_t *span_offset, const int64_t *span_bytes,
                    const int64_t *block_ids, const uint64_t *sources, size_t n_blocks)
{
    for (size_t i = 0; i < n_blocks; ++i)
        for (size_t s = 0; s < n_spans; ++s)
            memmove((uint8_t *)(uintptr_t)(span_base[s] + (uint64_t)(block_ids[i] * span_pitch[s])),
                    (const uint8_t *)(uintptr_t)(sources[i] + (uint64_t)span_offset[s]),
                    (size_t)span_bytes[s]);
}

/* _zero_tail, kvsnap/connector/dataplane.py:262-272: for each layer of one
 * packed record, every head h and token t in [valid, N) loses its C elements
 * at layer_offset + (h*sh + t*sn) * esize.  geometry[l] = {H, N, C, sh, sn,
 * esize}. */
void oracle_zero_tail(uint8_t *record, size_t n_layers, const int64_t *layer_offset,
                      const int64_t *geometry, int64_t valid)
{
    for (size_t l = 0; l < n_layers; ++l) {
        const int64_t *g = geometry + 6 * l;
        int64_t H = g[0], N = g[1], C = g[2], sh = g[3], sn = g[4], es = g[5];
        for (int64_t h = 0; h < H; ++h)
            for (int64_t t = valid; t < N; ++t)
                memset(record + layer_offset[l] + (h * sh + t * sn) * es, 0, (size_t)(C * es));
    }
}

/* ------------------------------------------------------------------------ */
/* Seeded synthetic KV (not a reference function: the bench's input).       */
/* Integer-only so that the GPU generator can match it bit for bit.          */
/* ------------------------------------------------------------------------ */

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t oracle_span_key(uint64_t seed, uint64_t span, uint64_t block)
{
    uint64_t h = mix64(seed + 0x9E3779B97F4A7C15ull);
    h = mix64(h + span * 0xD1B54A32D192ED03ull);
    return mix64(h + block * 0xABC98388FB8FAC03ull);
}

/* One element's ~N(0,1) sample as float: Irwin-Hall of four 16-bit uniforms,
 * centred and scaled by an fp32 multiply (exact integer -> float, one
 * correctly rounded product). */
static inline float normal_sample(uint64_t key, uint64_t element)
{
    uint64_t r = mix64(key + element * 0x9E3779B97F4A7C15ull);
    int32_t sum = (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) +
                  (int32_t)((r >> 32) & 0xFFFF) + (int32_t)(r >> 48);
    return (float)(sum - 131070) * 2.6429e-05f;
}

static inline uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

/* float -> bfloat16, round to nearest even (finite inputs only). */
static inline uint16_t to_bf16(float x)
{
    uint32_t u = f32_bits(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* float -> OCP fp8 e4m3fn, round to nearest even, saturating to +-448. */
static inline uint8_t to_e4m3(float x)
{
    uint32_t u = f32_bits(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x43E00000u) /* |x| >= 448 */
        return sign | 0x7E;
    if (a < 0x3C800000u) { /* |x| < 2^-6: subnormal grid of 2^-9 */
        /* value / 2^-9 rounded to nearest even, in [0, 8] */
        float v;
        memcpy(&v, &a, 4);
        float q = v * 512.0f;             /* exact: power-of-two scaling */
        uint32_t n = (uint32_t)q;         /* floor */
        float frac = q - (float)n;        /* exact for q < 8 */
        if (frac > 0.5f || (frac == 0.5f && (n & 1u)))
            ++n;
        return sign | (uint8_t)n;         /* n == 8 is the smallest normal */
    }
    /* normal: keep 3 mantissa bits, RNE on the remaining 20 */
    uint32_t rounded = a + 0x7FFFFu + ((a >> 20) & 1u);
    uint32_t exp = (rounded >> 23) - 127 + 7;
    uint32_t man = (rounded >> 20) & 7u;
    uint32_t code = (exp << 3) | man;
    if (code > 0x7E)
        code = 0x7E;
    return sign | (uint8_t)code;
}

/* Fill one span's bytes in storage order.  kind 0: bf16 N(0,1); kind 1:
 * fp8-e4m3 of N(0,1) * inv_scale; kind 2: raw random bytes. */
void oracle_fill_span(uint64_t seed, uint64_t span, uint64_t block, uint8_t *out, size_t bytes,
                      int kind, float inv_scale)
{
    uint64_t key = oracle_span_key(seed, span, block);
    if (kind == 0) {
        for (size_t e = 0; e < bytes / 2; ++e) {
            uint16_t v = to_bf16(normal_sample(key, e));
            memcpy(out + 2 * e, &v, 2);
        }
    } else if (kind == 1) {
        for (size_t e = 0; e < bytes; ++e)
            out[e] = to_e4m3(normal_sample(key, e) * inv_scale);
    } else {
        for (size_t e = 0; e < bytes / 8; ++e) {
            uint64_t r = mix64(key + e * 0x9E3779B97F4A7C15ull);
            memcpy(out + 8 * e, &r, 8);
        }
    }
}

uint16_t oracle_to_bf16(float x) { return to_bf16(x); }
uint8_t oracle_to_e4m3(float x) { return to_e4m3(x); }

/* ------------------------------------------------------------------------ */
/* Batched record digests on `threads` host threads (the CPU baseline:       */
/* volatile.py:229-232 and store.py:621-622 hash blocks on 8 threads).       */
/* ------------------------------------------------------------------------ */

struct digest_job {
    const uint8_t *base;
    size_t record_bytes, pitch, first, last;
    uint32_t *crc;
    uint8_t *sha;
};

static void *digest_worker(void *arg)
{
    struct digest_job *job = (struct digest_job *)arg;
    for (size_t i = job->first; i < job->last; ++i) {
        const uint8_t *rec = job->base + i * job->pitch;
        if (job->crc)
            job->crc[i] = oracle_crc32c(rec, job->record_bytes, 0);
        if (job->sha)
            oracle_sha256(rec, job->record_bytes, job->sha + 32 * i);
    }
    return NULL;
}

/* crc and/or sha may be NULL.  Returns 0 or -1 if a thread cannot start. */
int oracle_digest_records(const uint8_t *base, size_t record_bytes, size_t pitch, size_t n,
                          uint32_t *crc, uint8_t *sha, int threads)
{
    if (threads < 1)
        threads = 1;
    if (threads > 256)
        threads = 256;
    pthread_t tid[256];
    struct digest_job jobs[256];
    size_t per = (n + (size_t)threads - 1) / (size_t)threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        size_t first = (size_t)t * per, last = first + per > n ? n : first + per;
        jobs[t] = (struct digest_job){base, record_bytes, pitch, first < n ? first : n, last, crc, sha};
        if (pthread_create(&tid[t], NULL, digest_worker, &jobs[t]) != 0) {
            for (int j = 0; j < started; ++j)
                pthread_join(tid[j], NULL);
            return -1;
        }
        ++started;
    }
    for (int t = 0; t < started; ++t)
        pthread_join(tid[t], NULL);
    return 0;
}

struct copy_job {
    size_t n_spans;
    const uint64_t *span_base;
    const int64_t *span_pitch, *span_offset, *span_bytes, *block_ids;
    const uint64_t *sources;
    uint8_t *records;
    size_t block_bytes, first, last;
};

static void *gather_worker(void *arg)
{
    struct copy_job *j = (struct copy_job *)arg;
    if (j->last > j->first)
        oracle_gather(j->n_spans, j->span_base, j->span_pitch, j->span_offset, j->span_bytes,
                      j->block_ids + j->first, j->last - j->first, j->records + j->first * j->block_bytes,
                      j->block_bytes);
    return NULL;
}

static void *scatter_worker(void *arg)
{
    struct copy_job *j = (struct copy_job *)arg;
    if (j->last > j->first)
        oracle_scatter(j->n_spans, j->span_base, j->span_pitch, j->span_offset, j->span_bytes,
                       j->block_ids + j->first, j->sources + j->first, j->last - j->first);
    return NULL;
}

/* Threaded gather (sources == NULL) or scatter, split over blocks. */
int oracle_copy_threads(size_t n_spans, const uint64_t *span_base, const int64_t *span_pitch,
                        const int64_t *span_offset, const int64_t *span_bytes, const int64_t *block_ids,
                        const uint64_t *sources, size_t n_blocks, uint8_t *records, size_t block_bytes,
                        int threads)
{
    if (threads < 1)
        threads = 1;
    if (threads > 256)
        threads = 256;
    pthread_t tid[256];
    struct copy_job jobs[256];
    size_t per = (n_blocks + (size_t)threads - 1) / (size_t)threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        size_t first = (size_t)t * per, last = first + per > n_blocks ? n_blocks : first + per;
        if (first > n_blocks)
            first = n_blocks;
        jobs[t] = (struct copy_job){n_spans, span_base, span_pitch, span_offset, span_bytes, block_ids,
                                    sources, records, block_bytes, first, last};
        if (pthread_create(&tid[t], NULL, sources ? scatter_worker : gather_worker, &jobs[t]) != 0) {
            for (int j = 0; j < started; ++j)
                pthread_join(tid[j], NULL);
            return -1;
        }
        ++started;
    }
    for (int t = 0; t < started; ++t)
        pthread_join(tid[t], NULL);
    return 0;
}
