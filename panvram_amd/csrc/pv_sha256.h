// pv_sha256.h - SHA-256 (FIPS 180-4), host side. refrel3 v1 binds every archive to the decoded reference by the
// SHA-256 of its upper-case base stream (reference FORMAT.md section 1, header offset 24; checked at open,
// reference csrc/pv_core.cpp:40 and csrc/pv_v1.h:115). Pinned by the tests against Python's hashlib.
#pragma once
#include <stdint.h>
#include <string.h>
#include <dlfcn.h>
#include <stdlib.h>

namespace pvs {

// FIPS 180-4 section 4.2.2: first 32 bits of the fractional parts of the cube roots of the first 64 primes
static const uint32_t K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

static inline uint32_t ror(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }

struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint8_t buf[64]; uint32_t nbuf = 0; uint64_t total = 0;
    void block(const uint8_t* p) {
        uint32_t w[64];
        for (int t = 0; t < 16; t++) w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
        for (int t = 16; t < 64; t++) {
            const uint32_t s0 = ror(w[t - 15], 7) ^ ror(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = ror(w[t - 2], 17) ^ ror(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
        for (int t = 0; t < 64; t++) {
            const uint32_t t1 = k + (ror(e, 6) ^ ror(e, 11) ^ ror(e, 25)) + ((e & f) ^ (~e & g)) + K[t] + w[t];
            const uint32_t t2 = (ror(a, 2) ^ ror(a, 13) ^ ror(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            k = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += k;
    }
    void update(const uint8_t* p, uint64_t n) {
        total += n;
        if (nbuf) { const uint32_t k = (uint32_t)(n < 64 - nbuf ? n : 64 - nbuf); memcpy(buf + nbuf, p, k); nbuf += k; p += k; n -= k;
                    if (nbuf == 64) { block(buf); nbuf = 0; } }
        while (n >= 64) { block(p); p += 64; n -= 64; }
        if (n) { memcpy(buf, p, n); nbuf = (uint32_t)n; }
    }
    void digest(uint8_t out[32]) {
        const uint64_t bits = total * 8; uint8_t pad[72] = {0x80}; const uint32_t k = nbuf < 56 ? 56 - nbuf : 120 - nbuf;
        for (int i = 0; i < 8; i++) pad[k + i] = (uint8_t)(bits >> (56 - 8 * i));
        update(pad, k + 8);
        for (int i = 0; i < 8; i++) { out[4 * i] = (uint8_t)(h[i] >> 24); out[4 * i + 1] = (uint8_t)(h[i] >> 16); out[4 * i + 2] = (uint8_t)(h[i] >> 8); out[4 * i + 3] = (uint8_t)h[i]; }
    }
};

static inline void sha256_portable(const uint8_t* p, uint64_t n, uint8_t out[32]) { Sha256 s; s.update(p, n); s.digest(out); }

// SHA-256 through the system OpenSSL (libcrypto.so.3: SHA-NI / AVX2 code, ~10x the portable loop) when it can be
// loaded, else the portable implementation above. Same digest either way (both are FIPS 180-4).
static inline void sha256(const uint8_t* p, uint64_t n, uint8_t out[32]) {
    typedef unsigned char* (*Fn)(const unsigned char*, size_t, unsigned char*);
    static const Fn fn = []() -> Fn {
        if (getenv("PANVRAM_SHA256_PORTABLE")) return nullptr;      // force the portable path (its test)
        void* h = dlopen("libcrypto.so.3", RTLD_NOW | RTLD_LOCAL);
        return h ? (Fn)dlsym(h, "SHA256") : (Fn) nullptr;
    }();
    if (fn) fn(p, (size_t)n, out); else sha256_portable(p, n, out);
}

}  // namespace pvs
