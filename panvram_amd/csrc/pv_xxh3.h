// pv_xxh3.h - XXH3_64bits with seed 0 (xxHash 0.8 family, the hash refrel3 v1 uses for its header, per-block and
// FASTA checks: reference FORMAT.md "All integers little-endian. XXH3 = XXH3_64bits (xxHash 0.8, seed 0)").
//
// Written from the published xxHash 0.8 algorithm description: the short paths (0..16, 17..128, 129..240 bytes) and
// the long path (64-byte stripes accumulated into eight 64-bit lanes, scrambled every 1024 bytes, merged at the end).
// The 192-byte default secret and the primes are the published constants of that specification (they have to be the
// same bytes, or the hashes differ). One-shot and streaming forms; both are pinned by the tests against the Python
// `xxhash` package (an independent implementation) for every length 0..4096 and for random long inputs.
//
// The per-stripe step is additive within a 1024-byte block, which is what a parallel (GPU) evaluation of the long path
// exploits; the helpers below are __host__ __device__ so the kernels can share them.
#pragma once
#include <stdint.h>
#include <string.h>
#if defined(__AVX2__) && !defined(__HIP_DEVICE_COMPILE__)
#include <immintrin.h>
#define PVX_AVX2 1
#endif

#if defined(__HIPCC__)
#define PV_HD __host__ __device__
#else
#define PV_HD
#endif

namespace pvx {

static constexpr uint64_t P32_1 = 0x9E3779B1u, P32_2 = 0x85EBCA77u, P32_3 = 0xC2B2AE3Du;
static constexpr uint64_t P64_1 = 0x9E3779B185EBCA87ull, P64_2 = 0xC2B2AE3D27D4EB4Full, P64_3 = 0x165667B19E3779F9ull,
                          P64_4 = 0x85EBCA77C2B2AE63ull, P64_5 = 0x27D4EB2F165667C5ull;
static constexpr uint64_t MX1 = 0x165667919E3779F9ull, MX2 = 0x9FB21C651E98DF25ull;
static constexpr int SECRET_SIZE = 192, STRIPE = 64, STRIPES_PER_BLOCK = (SECRET_SIZE - STRIPE) / 8, BLOCK = STRIPE * STRIPES_PER_BLOCK;

// the default secret of the specification (one copy for the host, one in device constant memory)
#define PVX_SECRET_BYTES \
    0xb8, 0xfe, 0x6c, 0x39, 0x23, 0xa4, 0x4b, 0xbe, 0x7c, 0x01, 0x81, 0x2c, 0xf7, 0x21, 0xad, 0x1c, \
    0xde, 0xd4, 0x6d, 0xe9, 0x83, 0x90, 0x97, 0xdb, 0x72, 0x40, 0xa4, 0xa4, 0xb7, 0xb3, 0x67, 0x1f, \
    0xcb, 0x79, 0xe6, 0x4e, 0xcc, 0xc0, 0xe5, 0x78, 0x82, 0x5a, 0xd0, 0x7d, 0xcc, 0xff, 0x72, 0x21, \
    0xb8, 0x08, 0x46, 0x74, 0xf7, 0x43, 0x24, 0x8e, 0xe0, 0x35, 0x90, 0xe6, 0x81, 0x3a, 0x26, 0x4c, \
    0x3c, 0x28, 0x52, 0xbb, 0x91, 0xc3, 0x00, 0xcb, 0x88, 0xd0, 0x65, 0x8b, 0x1b, 0x53, 0x2e, 0xa3, \
    0x71, 0x64, 0x48, 0x97, 0xa2, 0x0d, 0xf9, 0x4e, 0x38, 0x19, 0xef, 0x46, 0xa9, 0xde, 0xac, 0xd8, \
    0xa8, 0xfa, 0x76, 0x3f, 0xe3, 0x9c, 0x34, 0x3f, 0xf9, 0xdc, 0xbb, 0xc7, 0xc7, 0x0b, 0x4f, 0x1d, \
    0x8a, 0x51, 0xe0, 0x4b, 0xcd, 0xb4, 0x59, 0x31, 0xc8, 0x9f, 0x7e, 0xc9, 0xd9, 0x78, 0x73, 0x64, \
    0xea, 0xc5, 0xac, 0x83, 0x34, 0xd3, 0xeb, 0xc3, 0xc5, 0x81, 0xa0, 0xff, 0xfa, 0x13, 0x63, 0xeb, \
    0x17, 0x0d, 0xdd, 0x51, 0xb7, 0xf0, 0xda, 0x49, 0xd3, 0x16, 0x55, 0x26, 0x29, 0xd4, 0x68, 0x9e, \
    0x2b, 0x16, 0xbe, 0x58, 0x7d, 0x47, 0xa1, 0xfc, 0x8f, 0xf8, 0xb8, 0xd1, 0x7a, 0xd0, 0x31, 0xce, \
    0x45, 0xcb, 0x3a, 0x8f, 0x95, 0x16, 0x04, 0x28, 0xaf, 0xd7, 0xfb, 0xca, 0xbb, 0x4b, 0x40, 0x7e,
static const uint8_t kSecret[SECRET_SIZE] = {PVX_SECRET_BYTES};
#if defined(__HIPCC__)
__device__ __constant__ static const uint8_t kSecretDev[SECRET_SIZE] = {PVX_SECRET_BYTES};
#endif

PV_HD static inline uint64_t ld64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }
PV_HD static inline uint32_t ld32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
PV_HD static inline uint64_t rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
PV_HD static inline uint64_t bswap64(uint64_t x) {
    x = ((x & 0x00FF00FF00FF00FFull) << 8) | ((x >> 8) & 0x00FF00FF00FF00FFull);
    x = ((x & 0x0000FFFF0000FFFFull) << 16) | ((x >> 16) & 0x0000FFFF0000FFFFull);
    return (x << 32) | (x >> 32);
}
// 64x64 -> 128 multiply, the two halves folded by xor
PV_HD static inline uint64_t mulfold(uint64_t a, uint64_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return (a * b) ^ __umul64hi(a, b);
#else
    const unsigned __int128 p = (unsigned __int128)a * b;
    return (uint64_t)p ^ (uint64_t)(p >> 64);
#endif
}
PV_HD static inline uint64_t avalanche3(uint64_t h) { h ^= h >> 37; h *= MX1; return h ^ (h >> 32); }
PV_HD static inline uint64_t avalanche64(uint64_t h) { h ^= h >> 33; h *= P64_2; h ^= h >> 29; h *= P64_3; return h ^ (h >> 32); }
PV_HD static inline uint64_t rrmxmx(uint64_t h, uint64_t len) {
    h ^= rotl(h, 49) ^ rotl(h, 24); h *= MX2; h ^= (h >> 35) + len; h *= MX2; return h ^ (h >> 28);
}
PV_HD static inline uint64_t mix16(const uint8_t* in, const uint8_t* sec) {
    return mulfold(ld64(in) ^ ld64(sec), ld64(in + 8) ^ ld64(sec + 8));
}

// ---- short inputs (seed 0)
PV_HD static inline uint64_t hash_short(const uint8_t* in, uint64_t len, const uint8_t* S) {
    if (len <= 16) {
        if (len > 8) {
            const uint64_t lo = ld64(in) ^ (ld64(S + 24) ^ ld64(S + 32));
            const uint64_t hi = ld64(in + len - 8) ^ (ld64(S + 40) ^ ld64(S + 48));
            return avalanche3(len + bswap64(lo) + hi + mulfold(lo, hi));
        }
        if (len >= 4) {
            const uint64_t v = (uint64_t)ld32(in + len - 4) + ((uint64_t)ld32(in) << 32);
            return rrmxmx(v ^ (ld64(S + 8) ^ ld64(S + 16)), len);
        }
        if (len) {
            const uint32_t c = ((uint32_t)in[0] << 16) | ((uint32_t)in[len >> 1] << 24) | (uint32_t)in[len - 1] | ((uint32_t)len << 8);
            return avalanche64((uint64_t)(c ^ (ld32(S) ^ ld32(S + 4))));
        }
        return avalanche64(ld64(S + 56) ^ ld64(S + 64));
    }
    uint64_t acc = len * P64_1;
    if (len <= 128) {
        if (len > 32) {
            if (len > 64) {
                if (len > 96) { acc += mix16(in + 48, S + 96); acc += mix16(in + len - 64, S + 112); }
                acc += mix16(in + 32, S + 64); acc += mix16(in + len - 48, S + 80);
            }
            acc += mix16(in + 16, S + 32); acc += mix16(in + len - 32, S + 48);
        }
        acc += mix16(in, S); acc += mix16(in + len - 16, S + 16);
        return avalanche3(acc);
    }
    // 129..240
    for (int i = 0; i < 8; i++) acc += mix16(in + 16 * i, S + 16 * i);
    uint64_t acc_end = mix16(in + len - 16, S + 136 - 17);
    acc = avalanche3(acc);
    const int rounds = (int)(len / 16);
    for (int i = 8; i < rounds; i++) acc_end += mix16(in + 16 * i, S + 16 * (i - 8) + 3);
    return avalanche3(acc + acc_end);
}

// ---- long inputs: 8 accumulator lanes
PV_HD static inline void acc_init(uint64_t acc[8]) {
    acc[0] = P32_3; acc[1] = P64_1; acc[2] = P64_2; acc[3] = P64_3; acc[4] = P64_4; acc[5] = P32_2; acc[6] = P64_5; acc[7] = P32_1;
}
PV_HD static inline void stripe(uint64_t acc[8], const uint8_t* in, const uint8_t* sec) {
    for (int i = 0; i < 8; i++) {
        const uint64_t d = ld64(in + 8 * i), k = d ^ ld64(sec + 8 * i);
        acc[i ^ 1] += d;
        acc[i] += (k & 0xFFFFFFFFull) * (k >> 32);
    }
}
PV_HD static inline void scramble(uint64_t acc[8], const uint8_t* sec) {
    for (int i = 0; i < 8; i++) { uint64_t a = acc[i]; a ^= a >> 47; a ^= ld64(sec + 8 * i); acc[i] = a * P32_1; }
}
PV_HD static inline uint64_t merge(const uint64_t acc[8], const uint8_t* sec, uint64_t start) {
    uint64_t r = start;
    for (int i = 0; i < 4; i++) r += mulfold(acc[2 * i] ^ ld64(sec + 16 * i), acc[2 * i + 1] ^ ld64(sec + 16 * i + 8));
    return avalanche3(r);
}
// `n` consecutive stripes, stripe s keyed by the secret at 8 s; then (if scr) the end-of-block scramble.
// Host builds with AVX2 process the eight lanes as two 256-bit vectors: lane i adds its data word to lane i^1 (a swap
// of the 64-bit halves of each 128-bit half) and lo32(key) * hi32(key) to itself - the same arithmetic.
#if defined(PVX_AVX2)
static inline void stripes_scramble(uint64_t acc[8], const uint8_t* in, const uint8_t* S, uint64_t n, bool scr) {
    __m256i a0 = _mm256_loadu_si256((const __m256i*)acc), a1 = _mm256_loadu_si256((const __m256i*)(acc + 4));
    for (uint64_t s = 0; s < n; s++) {
        const uint8_t* p = in + s * STRIPE; const uint8_t* k = S + 8 * s;
        const __m256i d0 = _mm256_loadu_si256((const __m256i*)p), d1 = _mm256_loadu_si256((const __m256i*)(p + 32));
        const __m256i k0 = _mm256_xor_si256(d0, _mm256_loadu_si256((const __m256i*)k));
        const __m256i k1 = _mm256_xor_si256(d1, _mm256_loadu_si256((const __m256i*)(k + 32)));
        a0 = _mm256_add_epi64(a0, _mm256_add_epi64(_mm256_mul_epu32(k0, _mm256_srli_epi64(k0, 32)), _mm256_shuffle_epi32(d0, _MM_SHUFFLE(1, 0, 3, 2))));
        a1 = _mm256_add_epi64(a1, _mm256_add_epi64(_mm256_mul_epu32(k1, _mm256_srli_epi64(k1, 32)), _mm256_shuffle_epi32(d1, _MM_SHUFFLE(1, 0, 3, 2))));
    }
    if (scr) {
        const __m256i P = _mm256_set1_epi64x((long long)P32_1);
        const uint8_t* k = S + SECRET_SIZE - STRIPE;
        __m256i* av[2] = {&a0, &a1};
        for (int h = 0; h < 2; h++) {
            __m256i a = *av[h];
            a = _mm256_xor_si256(_mm256_xor_si256(a, _mm256_srli_epi64(a, 47)), _mm256_loadu_si256((const __m256i*)(k + 32 * h)));
            const __m256i lo = _mm256_mul_epu32(a, P), hi = _mm256_mul_epu32(_mm256_srli_epi64(a, 32), P);
            *av[h] = _mm256_add_epi64(lo, _mm256_slli_epi64(hi, 32));
        }
    }
    _mm256_storeu_si256((__m256i*)acc, a0); _mm256_storeu_si256((__m256i*)(acc + 4), a1);
}
#else
PV_HD static inline void stripes_scramble(uint64_t acc[8], const uint8_t* in, const uint8_t* S, uint64_t n, bool scr) {
    for (uint64_t s = 0; s < n; s++) stripe(acc, in + s * STRIPE, S + 8 * s);
    if (scr) scramble(acc, S + SECRET_SIZE - STRIPE);
}
#endif

PV_HD static inline uint64_t hash_long(const uint8_t* in, uint64_t len, const uint8_t* S) {
    uint64_t acc[8]; acc_init(acc);
    const uint64_t nblocks = (len - 1) / BLOCK;
    for (uint64_t b = 0; b < nblocks; b++) stripes_scramble(acc, in + b * BLOCK, S, STRIPES_PER_BLOCK, true);
    const uint64_t ns = ((len - 1) - BLOCK * nblocks) / STRIPE;
    stripes_scramble(acc, in + nblocks * BLOCK, S, ns, false);
    stripe(acc, in + len - STRIPE, S + SECRET_SIZE - STRIPE - 7);
    return merge(acc, S + 11, len * P64_1);
}

PV_HD static inline uint64_t xxh3_64(const void* data, uint64_t len) {
    const uint8_t* in = (const uint8_t*)data;
#if defined(__HIP_DEVICE_COMPILE__)
    const uint8_t* S = kSecretDev;
#else
    const uint8_t* S = kSecret;
#endif
    return len <= 240 ? hash_short(in, len, S) : hash_long(in, len, S);
}

// ---- streaming (host): bytes arrive in pieces, the hash equals xxh3_64 of their concatenation.
// Whole 1024-byte blocks are consumed as soon as a later byte proves they are not the final block; the last
// up-to-1024 bytes (plus the 64 before them, for the final stripe) stay buffered until digest().
struct Stream {
    uint64_t acc[8];
    uint64_t total = 0;        // bytes seen
    uint8_t buf[BLOCK + STRIPE]; // buf[STRIPE ..] = pending bytes of the current block; buf[0, STRIPE) = tail of the previous block
    uint32_t nbuf = 0;         // pending bytes in buf[STRIPE ..]
    bool have_prev = false;    // a full block was consumed before (its last 64 bytes are in buf[0, STRIPE))
    uint8_t head[241];         // first bytes while total <= 240 (short path)
    Stream() { acc_init(acc); }
    void update(const void* data, uint64_t n) {
        const uint8_t* p = (const uint8_t*)data;
        while (n) {
            if (total < 241) { const uint64_t k = n < 241 - total ? n : 241 - total; memcpy(head + total, p, k); }
            if (nbuf == (uint32_t)BLOCK) {     // a byte follows a full pending block: that block is not the last one
                stripes_scramble(acc, buf + STRIPE, kSecret, STRIPES_PER_BLOCK, true);
                memcpy(buf, buf + BLOCK, STRIPE); nbuf = 0; have_prev = true;
            }
            if (nbuf == 0 && n > (uint64_t)BLOCK && total >= 241) {   // whole blocks straight from the input
                // every block except one that might be the last is consumed in place; its last 64 bytes are kept
                const uint64_t k = (n - 1) / BLOCK;
                for (uint64_t b = 0; b < k; b++) stripes_scramble(acc, p + b * BLOCK, kSecret, STRIPES_PER_BLOCK, true);
                memcpy(buf, p + k * BLOCK - STRIPE, STRIPE); have_prev = true;
                p += k * BLOCK; n -= k * BLOCK; total += k * BLOCK;
                continue;
            }
            const uint64_t k = n < (uint64_t)BLOCK - nbuf ? n : (uint64_t)BLOCK - nbuf;
            memcpy(buf + STRIPE + nbuf, p, k); nbuf += (uint32_t)k; total += k; p += k; n -= k;
        }
    }
    uint64_t digest() const {
        if (total <= 240) return hash_short(head, total, kSecret);
        uint64_t a[8]; memcpy(a, acc, sizeof a);
        // the pending bytes are the final (partial or full) block: its stripes except the last, then the last stripe
        const uint64_t ns = (nbuf - 1) / STRIPE;
        stripes_scramble(a, buf + STRIPE, kSecret, ns, false);
        uint8_t last[STRIPE];
        if (nbuf >= (uint32_t)STRIPE) memcpy(last, buf + STRIPE + nbuf - STRIPE, STRIPE);
        else { memcpy(last, buf + nbuf, STRIPE - nbuf); memcpy(last + STRIPE - nbuf, buf + STRIPE, nbuf); }  // tail of the previous block
        stripe(a, last, kSecret + SECRET_SIZE - STRIPE - 7);
        return merge(a, kSecret + 11, total * P64_1);
    }
};

}  // namespace pvx
