// pv_kernels.hip - refrel3 v1 window decode on MI355X (gfx950).
//
// A call's kernels, at block sizes up to 4096 with the light path on (the default):
//   calls of at most SMALL_SLOTS (16,384) slots: front_kernel - one wave per slot decodes a long payload into a heavy
//     area while one lane per slot decodes a short one into its slot record - then windows_kernel, which replays;
//   larger calls: slot_kernel (the slots' headers, and the heavy list, long payloads first), then heavy_kernel (wave k
//     decodes the list's k-th entry into heavy area k) beside light_decode_kernel (one lane per slot for the short
//     payloads), the two on two streams, then spill_kernel (the slots the areas or the slot records could not take,
//     whole), then windows_kernel with no decoder. Untimed on the caller's own stream, windows_kernel runs right after
//     the light lanes (beside the heavy waves) and leaves the heavy list's slots to the heavy waves themselves
//     (heavy_replay_fused_kernel: each wave replays the slot it decoded); spill_kernel follows the replay, then the
//     join.
// At block size 16384 (op lists in LDS) there are no heavy areas: a call of at most SMALL_SLOTS_Q16 (2,048) slots takes
// front_kernel's light lanes only (payloads of up to 64 bytes, one lane per slot) and windows_kernel's wave decoder for
// the rest; a larger call takes
// slot_kernel, light_decode_kernel, spill_kernel (every long block, whole) and the replay-only windows_kernel. With the
// light path off, windows_kernel does all of it, one slot per wave (below).
//
// windows_kernel: one 64-lane wavefront (one workgroup) per (window, covering block) slot:
//   1. stage: the 15 large-alphabet model rows into LDS, the 46 small-alphabet rows into VGPRs (lane i holds row i),
//      the rANS payload and the reference span the block's start diagonal predicts (plus a margin) into LDS;
//   2. decode the block's symbol stream - the serial part - with the rANS state wave-uniform: a 6-letter context by
//      a SWAR compare against its row, a 104-letter context by one LDS compare per lane and two ballots, long literal
//      runs two literals per step (16 lanes test the 16 symbol pairs at once, one v_readlane takes the winner);
//      literal bytes are gathered one per lane and stored 64 at a time, copies go to an LDS op list;
//   3. replay the copies the window needs (reference / reverse-complement / overlapping self copies), 64 lanes per op,
//      reading the staged reference span from LDS (other positions from HBM);
//   4. build the block's lower-case bitmask from the case runs, then write the window's part of the block to its
//      output row with lower case, reverse complement and tokens fused into the store.
//
// Semantics follow the reference: window -> covering blocks and status bits (csrc/pv_cuda.cu:38-85, run_windows
// :117-149), the block grammar (csrc/refrel3.h:114-160), copy execution (csrc/pv_v1.h:65-72), case runs
// (csrc/pv_cuda.cu:89-100) and the output transforms (csrc/pv_cuda.cu:101-112). Output bytes are identical to the
// reference CPU decoder's (csrc/pv_core.cpp:116-136) for every valid archive; a block that fails to decode sets
// status bit 1 and its slot writes nothing, as in the reference.
//
// Memory safety on corrupt input: payload reads stay inside [payload, payload + len) rounded up to 16 bytes (the
// device copy of the payload pool carries 1 KiB of padding), literal and copy destinations are bounded by the
// block length, reference reads by the reference length, self-copy sources by the block offset; every loop advances.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include "../../include/panvram_amd.h"
#include "pv_codec.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>
#include <algorithm>
#include <cstddef>
#include <atomic>
#include <chrono>
#include <mutex>
#include <thread>
#include <type_traits>
#include <vector>

namespace {

constexpr int WAVE = 64;
constexpr uint32_t RMARGIN = 256;        // reference bytes staged on each side of the start diagonal's span

template <int Q> struct Cfg {
    static constexpr uint32_t REFW = Q + 2 * RMARGIN + 32;           // staged reference span (+ alignment slack)
    static constexpr uint32_t MAXCOPY = Q / pvc::MIN_LEN + 1;        // copies per block: each >= 12 bases
    // a slot's small LDS area: a light slot's literal bytes, the 2-bit words of the reference span for a slot whose
    // block arrives decoded (its block buffer is taken), or for a block decoded here the rows of the 104-letter
    // contexts (+ 16 bytes of alignment slack)
    static constexpr uint32_t BIG_ROWS = pvc::NBIG * pvc::BIG_ROW * 2;
    static constexpr uint32_t AUX_A = BIG_ROWS + 16, AUX_B = REFW / 4 + 16;
    static constexpr uint32_t AUX = ((AUX_A > AUX_B ? AUX_A : AUX_B) + 15) & ~15u;
    // the op list lives in VGPRs (op k in lane k % 64 of register k / 64) up to q4k, in LDS beyond
    static constexpr bool REGOPS = Q <= 4096;
    static constexpr int NOPR = REGOPS ? (int)((MAXCOPY + WAVE - 1) / WAVE) : 1;
};

template <int Q> struct __align__(16) Lds {
    static constexpr bool SPAN = true;
    static constexpr bool WIN = false;                // blk and lower cover the whole block
    uint8_t blk[Q];                                   // the block, upper case
    uint8_t refw[Cfg<Q>::REFW];                       // reference [wbase, wbase + REFW)
    uint8_t aux[Cfg<Q>::AUX];                         // literal bytes and chunk list, or packed reference words
    uint32_t ops[Cfg<Q>::REGOPS ? 1 : Cfg<Q>::MAXCOPY][2];   // copy ops (LDS form): src, dst | len << 15 | kind << 30
    uint32_t lower[Q / 32];                           // lower-case bitmask of the block
};
// The replay-only windows kernel's LDS where the reference is held as bytes: the block and its case bitmask only (4.6
// KB at q4k against 10.4): the reference and a light slot's literal bytes are read from HBM and L2 where a copy needs
// them (16 bytes per lane), so twice as many waves fit on a CU. The kernel's time follows its occupancy - it waits on
// memory - until HBM bounds it.
// Where ops live in LDS (Q = 16384) this kernel replays only light slots (a long block there is done whole by
// spill_kernel), whose ops are at most a slot record's LITE_OPS. There, for windows of at most WIN_W bases, blk and
// lower hold only the window's part of the block, from the 32-byte boundary at or below its start; such a kernel
// replays light slots without self copies only (the light lanes leave those at Q = 16384 to the whole-slot pass). A
// launch allocates only what the call's W needs: the ops, then the block buffer (win_bytes: W + 64, rounded to 32),
// then its case bitmask right after it (lower_words), 6.2 KB at W = 5,000 against 9.8 at W = 8,192 and 18.9 for a
// whole block. The replay waits on memory, so its time follows the workgroups per CU that LDS allows (config 3's
// replay, W = 5,000: 426 us with a buffer for 8,192 bases, 343 us with one sized for W).
constexpr uint32_t LITE_OPS = 64;
constexpr uint32_t WIN_W = 8192, WIN_BYTES = WIN_W + 64;     // window part + 31 below + 16 of the last chunk, rounded
static_assert(WIN_BYTES % 32 == 0, "window buffer");
__host__ __device__ constexpr uint32_t win_bytes(uint32_t W) { return (W + 64 + 31) & ~31u; }
static_assert(win_bytes(WIN_W) == WIN_BYTES, "window buffer");
__host__ __device__ constexpr uint32_t lower_words(uint32_t W) { return (win_bytes(W) / 32 + 3) & ~3u; }   // 16-byte multiple
template <int Q, bool WINDOW = false> struct __align__(16) LdsLite {
    static constexpr bool SPAN = false;
    static constexpr bool WIN = false;
    static constexpr uint32_t BLK = (uint32_t)Q;
    uint8_t blk[BLK];
    uint32_t ops[Cfg<Q>::REGOPS ? 1 : LITE_OPS][2];
    uint32_t lower[BLK / 32];
};
// (the decoder's windows kernel replays a light slot in this layout, over its own LDS)
static_assert(sizeof(LdsLite<1024>) <= sizeof(Lds<1024>) && sizeof(LdsLite<2048>) <= sizeof(Lds<2048>) &&
              sizeof(LdsLite<4096>) <= sizeof(Lds<4096>) && sizeof(LdsLite<16384>) <= sizeof(Lds<16384>), "light layout");
template <int Q> struct __align__(16) LdsLite<Q, true> {
    static constexpr bool SPAN = false;
    static constexpr bool WIN = true;
    static constexpr uint32_t BLK = WIN_BYTES;                    // the largest window buffer: loop bounds
    uint32_t ops[Cfg<Q>::REGOPS ? 1 : LITE_OPS][2];
    alignas(16) uint8_t blk[BLK];                                  // allocated up to win_bytes(W), the bitmask after it
};
// the case bitmask of the block buffer: a member, or in the window kernel the words right after win_bytes(W)
template <class LS> __device__ __forceinline__ uint32_t* lower_of(LS& S, uint32_t) { return S.lower; }
template <int Q> __device__ __forceinline__ uint32_t* lower_of(LdsLite<Q, true>& S, uint32_t W) { return (uint32_t*)(S.blk + win_bytes(W)); }

// Where the wave decoder keeps the block it decodes: the slot's LDS (G = false, windows_kernel), or global memory (G =
// true, the heavy role of the front kernel, which has no LDS: the block goes to the slot's area in the work buffer).
// The rows of the 104-letter contexts: staged in the slot's LDS (G = false), read from the model table (G = true).
template <int Q, bool G> struct DecMem {
    Lds<Q>* S;
    uint8_t* blk;
    const uint16_t* big;
};

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x; }   // one wavefront per workgroup
__device__ __forceinline__ uint32_t rdl(uint32_t v, uint32_t lane) { return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)lane); }
__device__ __forceinline__ uint32_t rfl(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ uint32_t wrl(uint32_t old, uint32_t v, uint32_t lane) { return lane_id() == lane ? v : old; }   // compare + select
// the first lane of a 64-bit value, as a scalar
__device__ __forceinline__ int64_t rfl64(int64_t v) {
    return (int64_t)(((uint64_t)rfl((uint32_t)((uint64_t)v >> 32)) << 32) | rfl((uint32_t)v));
}
__device__ __forceinline__ int64_t rdl64(int64_t v, uint32_t lane) {
    return (int64_t)(((uint64_t)rdl((uint32_t)((uint64_t)v >> 32), lane) << 32) | rdl((uint32_t)v, lane));
}

// all lanes copy 16-byte aligned chunks covering [g, g + len) into dst (LDS, 16-byte aligned), at most cap bytes, with
// direct global-to-LDS loads (global_load_lds_dwordx4: lane i's 16 bytes land at the instruction's LDS base + 16 i, no
// VGPR round trip), so the staging copies of a slot are all in flight together. The caller waits for them
// (stage_wait) before reading dst. Returns g's offset inside dst. Source arrays carry >= 16 bytes of padding.
// STREAM: the cache policy of data read once (the reference span): non-temporal, so that streaming it through L2 does
// not evict what many slots share there (model tables, block tables, contig tables)
typedef __attribute__((address_space(3))) void* lds_ptr_t;
constexpr int KEEP = 0, STREAM = 2;
template <int POLICY = KEEP>
__device__ __forceinline__ uint32_t stage(uint8_t* dst, const uint8_t* g, uint32_t len, uint32_t cap) {
    const uint8_t* a = (const uint8_t*)((uintptr_t)g & ~(uintptr_t)15);
    const uint32_t mis = (uint32_t)((uintptr_t)g & 15);
    uint32_t nch = (mis + len + 15) / 16; if (nch > cap / 16) nch = cap / 16;
    const uint32_t l = lane_id();
    for (uint32_t c0 = 0; c0 < nch; c0 += WAVE) {
        const uint32_t c = c0 + l;
        if (c < nch) __builtin_amdgcn_global_load_lds((const void*)(a + (size_t)c * 16), (lds_ptr_t)(dst + c0 * 16), 16, 0, POLICY);
    }
    return mis;
}
// every staging copy issued so far has landed in LDS (then a barrier makes it visible to the wave's later reads)
__device__ __forceinline__ void stage_wait() { __builtin_amdgcn_s_waitcnt(0); __syncthreads(); }

// ---- rANS decoder state: wave-uniform scalars. Payload bytes come through a 64-bit scalar bit-buffer refilled four
// bytes at a time from the LDS copy of the payload (bytes past the staged cap from HBM).
struct Dec {
    uint32_t x;              // state
    uint32_t p, n;           // payload bytes consumed, payload length
    uint64_t buf;            // the next `cnt` payload bytes, first in the low byte
    uint32_t cnt;
    uint32_t q;              // payload index of the first byte not yet in buf (= p + cnt)
    const uint8_t* g;        // payload in HBM
    bool bad;
};
// four payload bytes starting at payload index q, as one little-endian word, through the scalar cache (the address is
// wave-uniform; the pool is padded past its end)
__device__ __forceinline__ uint32_t pay4(const Dec& d, uint32_t q) {
    const uintptr_t A = (uintptr_t)(d.g + q);
    const __attribute__((address_space(4))) uint32_t* w = (const __attribute__((address_space(4))) uint32_t*)(A & ~(uintptr_t)3);
    return (uint32_t)(((((uint64_t)w[1]) << 32) | w[0]) >> (8 * (A & 3)));
}
__device__ __forceinline__ void refill(Dec& d) { d.buf |= (uint64_t)pay4(d, d.q) << (8 * d.cnt); d.cnt += 4; d.q += 4; }
// x < 2^16 after a symbol or a raw-bit step: at most two payload bytes bring it back into [2^16, 2^24)
__device__ __forceinline__ void renorm(Dec& d) {
    if (d.x >= pvc::RANS_L) return;
    if (d.cnt < 2) refill(d);
    if (d.p >= d.n) { d.bad = true; return; }
    d.x = (d.x << 8) | (uint32_t)(d.buf & 0xFF); d.buf >>= 8; d.cnt--; d.p++;
    if (d.x >= pvc::RANS_L) return;
    if (d.p >= d.n) { d.bad = true; return; }
    d.x = (d.x << 8) | (uint32_t)(d.buf & 0xFF); d.buf >>= 8; d.cnt--; d.p++;
}
// small rows in VGPRs: lane i holds row i as (cum1 | cum2 << 16, cum3 | cum4 << 16, cum5 | cum6 << 16)
struct Small { uint32_t a, b, c; };
// One symbol of a <= 6-letter context, branch-free on the scalar unit. With X = cum1..cum4 as 16-bit fields, the
// symbol is the number of boundaries <= slot: a 64-bit SWAR compare ((slot x 4) | 0x8000.. - X keeps bit 15 of a
// field set iff slot >= that boundary) plus one compare for cum5. cum[s] and cum[s+1] are 16-bit fields of
// T0 = (0, cum1, cum2, cum3) and T1 = (cum4, cum5, cum6) picked by 64-bit shifts.
__device__ __forceinline__ uint32_t sym_small(Dec& d, const Small& R, uint32_t row) {
    const uint32_t a = rdl(R.a, row), b = rdl(R.b, row), c = rdl(R.c, row);
    const uint64_t X = (uint64_t)a | ((uint64_t)b << 32);
    const uint32_t x = rfl(d.x), slot = x & (pvc::M - 1);
    const uint32_t rep = slot * 0x10001u;
    const uint64_t H = 0x8000800080008000ull;
    const uint64_t m = ((((uint64_t)rep << 32) | rep | H) - X) & H;
    const uint32_t s = (uint32_t)__popcll(m) + ((((slot | 0x8000u) - (c & 0xFFFFu)) >> 15) & 1u);
    const uint64_t T0 = X << 16, T1 = (X >> 48) | ((uint64_t)c << 16);
    const uint32_t lo = (uint32_t)(s < 4 ? (T0 >> (16 * s)) : (T1 >> (16 * (s - 4)))) & 0xFFFFu;
    const uint32_t hi = (uint32_t)(s < 3 ? (T0 >> (16 * (s + 1))) : (T1 >> (16 * (s - 3)))) & 0xFFFFu;
    const uint32_t f = hi - lo;
    if (!f) { d.bad = true; return s; }
    d.x = f * (x >> pvc::PROB_BITS) + slot - lo;
    renorm(d);
    return s;
}
// Literal triples. Lane l stands for the symbol triple (s1, s2, s3) = (l >> 4, (l >> 2) & 3, l & 3) and holds, for each
// of the 16 order-2 literal contexts r, (lo | (freq - 4096) << 16) of s1 in context r (low half of AB[r]) and of s2 in
// the context after s1 (high half), and (C) of s3 in the context after s1 s2, which does not depend on r. All come from
// the model table's pair section, loaded on a block's first long literal run; AB is indexed by the wave-uniform
// context, which the compiler turns into one indexed move of a register pair.
typedef uint64_t v16ul __attribute__((ext_vector_type(16)));
// count of leading zeros (32 for 0; only lanes whose hypothesis fails can see 0)
__device__ __forceinline__ uint32_t ffbh(uint32_t v) { uint32_t r; asm("v_ffbh_u32 %0, %1" : "=v"(r) : "v"(v)); return r; }

// 104-letter context: lane l compares cum[l+1] and cum[l+65] (LDS); the symbol is the count of boundaries <= slot
template <int Q, bool G> __device__ __forceinline__ uint32_t sym_big(const DecMem<Q, G>& M, Dec& d, uint32_t row) {
    const uint32_t l = lane_id();
    const uint16_t* r = M.big + row * pvc::BIG_ROW;   // the context's row
    const uint32_t a = r[l + 1];
    const uint32_t b = (l + 65 <= (uint32_t)pvc::BIG_ALPHA) ? (uint32_t)r[l + 65] : 0xFFFFu;
    d.x = rfl(d.x);
    const uint32_t slot = d.x & (pvc::M - 1);
    const uint64_t m0 = __ballot(a <= slot && l + 1 < (uint32_t)pvc::BIG_ALPHA);
    const uint64_t m1 = __ballot(b <= slot && l + 65 < (uint32_t)pvc::BIG_ALPHA);
    const uint32_t s = rfl((uint32_t)(__popcll(m0) + __popcll(m1)));
    const uint32_t lo = s == 0 ? 0u : (s <= 64 ? rdl(a, s - 1) : rdl(b, s - 65));
    const uint32_t hi = s + 1 <= 64 ? rdl(a, s) : rdl(b, s - 64);
    const uint32_t f = hi - lo;
    if (!f) { d.bad = true; return s; }
    d.x = f * (d.x >> pvc::PROB_BITS) + slot - lo;
    renorm(d);
    return s;
}
// raw bits, <= 16 per step, low chunk first (csrc/refrel3.h:83-90)
__device__ __forceinline__ uint64_t draw(Dec& d, uint32_t nb) {
    uint64_t v = 0; uint32_t sh = 0;
    while (nb && !d.bad) {
        const uint32_t k = nb > 16 ? 16 : nb;
        const uint32_t b = d.x & ((1u << k) - 1); d.x >>= k;
        renorm(d);
        v |= (uint64_t)b << sh; sh += k; nb -= k;
    }
    return v;
}
template <int Q, bool G> __device__ __forceinline__ uint64_t dval_big(const DecMem<Q, G>& M, Dec& d, uint32_t row) {
    const uint32_t s = sym_big(M, d, row);
    if (d.bad) return 0;
    return pvc::unbucket(s, draw(d, pvc::nbits_of(s)));
}

// small-row and big-row indices (pv_codec.h layout: small rows in context order LITR..KIND, REPK, DIR, FLIPK)
constexpr uint32_t SR_LITR = 0, SR_LIT2 = pvc::C_LIT2 - pvc::C_LITR, SR_KIND = pvc::C_KIND - pvc::C_LITR, SR_REPK = 43, SR_DIR = 44, SR_FLIPK = 45;
constexpr uint32_t BR_LL = 0, BR_DELTA = 4, BR_REPD = 6, BR_SELF = 7, BR_LEN = 8, BR_FLIPD = 14;
static_assert(pvc::row_of(pvc::C_REPK) == SR_REPK * pvc::SMALL_ROW && pvc::row_of(pvc::C_FLIPK) == SR_FLIPK * pvc::SMALL_ROW, "small rows");
static_assert(pvc::row_of(pvc::C_KIND + 15) == (SR_KIND + 15) * pvc::SMALL_ROW, "small rows");
static_assert(pvc::row_of(pvc::C_LL + 3) == pvc::SMALL_BYTES / 2 + 3 * pvc::BIG_ROW, "big rows");
static_assert(pvc::row_of(pvc::C_DELTA + 1) == pvc::SMALL_BYTES / 2 + (BR_DELTA + 1) * pvc::BIG_ROW, "big rows");
static_assert(pvc::row_of(pvc::C_REPD) == pvc::SMALL_BYTES / 2 + BR_REPD * pvc::BIG_ROW, "big rows");
static_assert(pvc::row_of(pvc::C_SELF) == pvc::SMALL_BYTES / 2 + BR_SELF * pvc::BIG_ROW, "big rows");
static_assert(pvc::row_of(pvc::C_LEN + 5) == pvc::SMALL_BYTES / 2 + (BR_LEN + 5) * pvc::BIG_ROW, "big rows");
static_assert(pvc::row_of(pvc::C_FLIPD) == pvc::SMALL_BYTES / 2 + BR_FLIPD * pvc::BIG_ROW, "big rows");

// reference view: a staged span in LDS, HBM elsewhere - the byte array, or in the packed form the 2-bit words and the
// runs of other bytes
struct RefView {
    const uint8_t* g; uint64_t n; int64_t wbase; uint32_t wlen;
    const uint32_t* pw; const int64_t* pes; const int64_t* pel; const uint8_t* peb; const uint32_t* peix; int64_t pne;
};
constexpr uint32_t ACGT = 'A' | ('C' << 8) | ('G' << 16) | ('T' << 24);
// byte q of the packed reference: a run of another byte holding q, else the word's 2-bit code. The bucket index gives
// the first run ending after the bucket start; runs are sorted and disjoint, so the scan stops at the first run
// starting after q.
__device__ __forceinline__ uint8_t packed_at(const RefView& R, uint64_t q) {
    for (int64_t r = R.peix[q >> PV_EXC_BUCKET_BITS]; r < R.pne; r++) {
        const uint64_t rs = (uint64_t)R.pes[r];
        if (rs > q) break;
        if (q < rs + (uint64_t)R.pel[r]) return R.peb[r];
    }
    return (uint8_t)(ACGT >> (8 * ((R.pw[q >> 4] >> (2 * (q & 15))) & 3)));
}
template <int Q> __device__ __forceinline__ uint8_t ref_at(const Lds<Q>& S, const RefView& R, uint64_t q) {
    const uint64_t k = q - (uint64_t)R.wbase;
    if (k < R.wlen) return S.refw[k];
    return R.pw ? packed_at(R, q) : R.g[q];
}
template <int Q, bool WINDOW> __device__ __forceinline__ uint8_t ref_at(const LdsLite<Q, WINDOW>&, const RefView& R, uint64_t q) {
    return R.pw ? packed_at(R, q) : R.g[q];
}
// the same for the wave decoder's memory: a 32-bit LDS read of the staged span (or a byte from HBM) - different load
// widths keep the two paths from being merged into one generic (flat) load
template <int Q, bool G> __device__ __forceinline__ uint32_t ref_at_v(const DecMem<Q, G>& M, const RefView& R, uint64_t q) {
    if constexpr (!G) {
        const uint64_t k = q - (uint64_t)R.wbase;
        if (k < R.wlen) return (((const uint32_t*)M.S->refw)[k >> 2] >> (8 * (k & 3))) & 0xFF;
    }
    return R.pw ? packed_at(R, q) : R.g[q];
}
// base code of a reference byte (A0 C1 G2 T3, other 4), complemented on the reverse strand, without branches
__device__ __forceinline__ uint32_t base_code(uint32_t b, uint32_t dir) {
    uint32_t r = 4;
    r = b == 'A' ? 0 : r; r = b == 'C' ? 1 : r; r = b == 'G' ? 2 : r; r = b == 'T' ? 3 : r;
    return (dir && r < 4) ? 3 - r : r;
}

// the four-entry move-to-front diagonal cache (csrc/refrel3.h:94-102), one entry per lane: lane k < n holds entry k
// (the diagonal as two words, and its strand). A push compares every entry at once (one ballot) and moves entries
// 0 .. j-1 up by one with a lane shift, where scalar registers would take a chain of compares and selects and, beside
// the rest of the decoder's wave-uniform state, more scalar registers than a wave has.
// lane i takes v of lane i - 1 (lanes 1 .. 15 of each row of 16; the others keep theirs)
__device__ __forceinline__ uint32_t lane_up(uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x111, 0xF, 0xF, false); }
struct Cache {
    uint32_t lo, hi, dir;     // lane k: entry k
    uint32_t n;               // entries held (1 .. 4)
    __device__ __forceinline__ void init(int64_t c0, uint32_t d0) {
        const bool z = lane_id() == 0;
        lo = z ? (uint32_t)c0 : 0u; hi = z ? (uint32_t)((uint64_t)c0 >> 32) : 0u; dir = z ? d0 : 0u; n = 1;
    }
    __device__ __forceinline__ int64_t cc(uint32_t k) const { return (int64_t)(((uint64_t)rdl(hi, k) << 32) | rdl(lo, k)); }
    __device__ __forceinline__ uint32_t dd(uint32_t k) const { return rdl(dir, k); }
    __device__ __forceinline__ void push(int64_t gc, uint32_t gd) {
        const uint32_t l = lane_id(), glo = (uint32_t)gc, ghi = (uint32_t)((uint64_t)gc >> 32);
        const uint64_t m = __ballot(l < n && lo == glo && hi == ghi && dir == gd);
        uint32_t j;
        if (m) {
            j = (uint32_t)__builtin_ctzll(m);                  // the first entry equal to the new one
        } else {
            if (n < 4) n++;
            j = n - 1;                                          // none: the last entry drops out (or a free one is taken)
        }
        const uint32_t ulo = lane_up(lo), uhi = lane_up(hi), ud = lane_up(dir);
        const bool up = l <= j;
        lo = l == 0 ? glo : up ? ulo : lo;
        hi = l == 0 ? ghi : up ? uhi : hi;
        dir = l == 0 ? gd : up ? ud : dir;
    }
};

// the op list in VGPRs: op k is lane k % 64 of element k / 64 of a register vector, indexed with the wave-uniform k / 64
// (an indexed register move; NOPR <= 8 for the block sizes that use it)
typedef uint32_t v8u __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
// 16 bytes from global memory at any byte address (one 16-byte load)
__device__ __forceinline__ v4u gload16(const uint8_t* p) {
    v4u v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
template <int Q> struct OpRegs { v8u src, w1; };
static_assert(Cfg<4096>::NOPR <= 8, "op registers");
template <int Q> __device__ __forceinline__ void op_put(OpRegs<Q>& R, uint32_t k, uint32_t src, uint32_t w1) {
    const bool me = lane_id() == (k & (WAVE - 1));
    switch (rfl(k / WAVE)) {            // wave-uniform: a scalar branch to a write with a constant index
#define PV_OPCASE(t) case t: R.src[t] = me ? src : R.src[t]; R.w1[t] = me ? w1 : R.w1[t]; break;
        PV_OPCASE(0) PV_OPCASE(1) PV_OPCASE(2) PV_OPCASE(3) PV_OPCASE(4) PV_OPCASE(5) PV_OPCASE(6) PV_OPCASE(7)
#undef PV_OPCASE
        default: break;
    }
}
__device__ __forceinline__ uint32_t op_get(const v8u& a, uint32_t k) { return rdl(a[rfl(k / WAVE) & 7], k & (WAVE - 1)); }

// literal bytes, one per lane, stored 64 at a time
template <int Q, bool G> __device__ __forceinline__ void blk_put(const DecMem<Q, G>& M, uint32_t i, uint8_t v) {
    if constexpr (G) M.blk[i] = v; else M.S->blk[i] = v;
}
struct LitAcc {
    uint32_t v; uint32_t base; uint32_t k;            // bytes for block positions base .. base + k - 1 in lanes 0 .. k-1
    template <int Q, bool G> __device__ __forceinline__ void flush(const DecMem<Q, G>& M) {
        if (k) { if (lane_id() < k) blk_put(M, base + lane_id(), (uint8_t)v); base += k; k = 0; }
    }
    template <int Q, bool G> __device__ __forceinline__ void put(const DecMem<Q, G>& M, uint32_t byte) {
        v = wrl(v, byte, k); k++;
        if (k == WAVE) flush(M);
    }
};

// decode one block into S.blk (literals) and S.ops (copies). Returns the number of copy ops, or -1 on failure
// (csrc/refrel3.h:114-160; every failure condition of the reference fails here too).
template <int Q, bool G> __device__ __forceinline__ int decode_block(const DecMem<Q, G>& S, OpRegs<Q>& OP, Dec& d, const Small& SR, const uint8_t* gtab,
                                                          const RefView& R, uint32_t blen, int64_t c0, uint32_t dir0) {
    Cache C; C.init(c0, dir0);
    int prevk = -1; uint32_t o = 0; int nops = 0;
    LitAcc lit; lit.v = 0; lit.k = 0; lit.base = 0;
    v16ul AB; uint32_t PC = 0; bool pready = false;      // literal-triple tables, loaded on the first long run
    constexpr uint32_t ACGTN = 'A' | ('C' << 8) | ('G' << 16) | ('T' << 24);
    while (o < blen) {
        o = rfl(o); prevk = (int)rfl((uint32_t)prevk); nops = (int)rfl((uint32_t)nops);
        C.n = rfl(C.n);
        const uint64_t ll = dval_big(S, d, BR_LL + pvc::kclass(prevk));
        if (d.bad || ll > blen - o) return -1;
        if (ll) {
            lit.base = o; lit.k = 0;
            if (ll <= 8) {
                // short run: context = the reference base the current diagonal predicts, x2, + first literal. Lane j
                // finds literal j's base (all at once: one read each), the serial loop takes it with a lane read.
                uint32_t rbl = 4;
                {
                    const int64_t c0 = C.cc(0); const uint32_t d0 = C.dd(0);
                    const int64_t q = pvc::diag_locus(c0, d0, o + lane_id());
                    if (lane_id() < (uint32_t)ll && q >= 0 && (uint64_t)q < R.n) rbl = base_code(ref_at_v(S, R, (uint64_t)q), d0);
                }
                for (uint32_t j = 0; j < (uint32_t)ll; j++) {
                    const uint32_t rb = rdl(rbl, j);
                    const uint32_t s = sym_small(d, SR, SR_LITR + rb * 2 + (j == 0 ? 1 : 0));
                    if (d.bad) return -1;
                    uint32_t byte = s < 4 ? (ACGTN >> (8 * s)) & 0xFF : 'N';
                    if (s == 5) { byte = (uint32_t)draw(d, 8); if (d.bad) return -1; }
                    lit.put(S, byte);
                }
            } else {
                // long run: order-2 context on the run's own literals (first: 16, then (previous * 4 + this) & 15).
                // The first literal takes the general path; then groups of eight literal pairs, then the general path.
                uint32_t r = 16, j = 0;
                {
                    const uint32_t s = sym_small(d, SR, SR_LIT2 + 16);
                    if (d.bad) return -1;
                    uint32_t byte = s < 4 ? (ACGTN >> (8 * s)) & 0xFF : 'N';
                    if (s == 5) { byte = (uint32_t)draw(d, 8); if (d.bad) return -1; }
                    lit.put(S, byte); lit.flush(S);
                    r = s < 4 ? s : 0; j = 1;
                }
                // Triple steps: every lane decodes its triple (s1, s2, s3) from the current state as if it were right -
                // symbol step, renormalisation (its byte count from the leading zeros, the bytes from the big-endian
                // window V of buffered payload), and so on for s2 and s3, each in the context its predecessors lead
                // to - and checks that all three slots fall in its symbols' ranges. Exactly one lane passes when the
                // three literals are A/C/G/T; its index holds the next context and v_readlane takes its state and byte
                // count. A group of five triples commits when all found a lane and the bytes they read were buffered
                // and inside the payload; otherwise its fifteen literals are decoded again on the general path (the
                // state is untouched).
                constexpr uint32_t G3 = 5;                   // triples per commit: 15 literals, 30 bits of codes
                if (j + 3 * G3 <= (uint32_t)ll && !pready) {
                    // lane l = 16 s1 + 4 s2 + s3: s1 in the run's context r and s2 in the context after s1 from the pair
                    // section's entry (r, l >> 2); s3 in context (l >> 2) = 4 s1 + s2, the pair section's first entry
                    // of that context for symbol l & 3
                    const uint2* src = (const uint2*)(gtab + pvc::PAIR_OFF);
                    const uint32_t pl = lane_id() >> 2;
#pragma unroll
                    for (int k = 0; k < 16; k++) { const uint2 e = src[16 * k + pl]; AB[k] = (uint64_t)e.x | ((uint64_t)e.y << 32); }
                    PC = src[16 * pl + 4 * (lane_id() & 3)].x;
                    pready = true;
                }
                while (j + 3 * G3 <= (uint32_t)ll) {
                    // groups on the triple path while they commit; a group that does not (an N or escape literal
                    // among its fifteen, or bytes past the buffer) leaves this loop for the general path below. The
                    // loop has one exit and no early return, so that the compiler keeps it tight (merged into the
                    // decoder's outer loop it took 112 instead of 100 clocks per literal).
                    bool stalled = false;
                    do {
                        if (d.cnt <= 4) refill(d);
                        uint64_t V = __builtin_bswap64(d.buf);       // buffered bytes, first in the top byte (zeros past cnt)
                        uint32_t x = d.x, bits = 0, orL = 0, acc = 0, rr = rfl(r);
#pragma unroll
                        for (uint32_t u = 0; u < G3; u++) {
                            const uint64_t ab = AB[rr & 15];
                            const uint32_t a = (uint32_t)ab, b = (uint32_t)(ab >> 32);
                            // With F = freq - 4096: F (x >> 12) + (x - lo) = freq (x >> 12) + (x & 4095) - lo, the decode step,
                            // and x's slot is in [lo, lo + freq) iff ((x - lo) & 4095) - 4096 < F (lo + freq <= 4096).
                            // Renormalisation: the state's leading zeros give the payload bits it takes (0, 8 or 16), and a
                            // 64-bit shift of (state, next payload word) by that many moves them in.
                            const int32_t Fa = (int32_t)a >> 16;
                            const uint32_t u1 = x - (a & 0xFFFF);
                            const uint64_t m1 = __ballot((int32_t)(u1 | 0xFFFFF000u) < Fa);
                            const uint32_t y = (uint32_t)(__mul24(Fa, (int32_t)(x >> pvc::PROB_BITS)) + (int32_t)u1);
                            const uint32_t s1 = (ffbh(y) - 8) & 24;
                            const uint32_t y1 = (uint32_t)(((((uint64_t)y << 32) | (uint32_t)(V >> 32)) << s1) >> 32);
                            const uint64_t Vb = V << s1;                              // window after those bytes
                            const int32_t Fb = (int32_t)b >> 16;
                            const uint32_t u2 = y1 - (b & 0xFFFF);
                            const uint64_t m2 = __ballot((int32_t)(u2 | 0xFFFFF000u) < Fb);
                            const uint32_t z = (uint32_t)(__mul24(Fb, (int32_t)(y1 >> pvc::PROB_BITS)) + (int32_t)u2);
                            const uint32_t s2 = (ffbh(z) - 8) & 24;
                            const uint32_t z1 = (uint32_t)(((((uint64_t)z << 32) | (uint32_t)(Vb >> 32)) << s2) >> 32);
                            const uint64_t Vc = Vb << s2;
                            const int32_t Fc = (int32_t)PC >> 16;
                            const uint32_t u3 = z1 - (PC & 0xFFFF);
                            const uint64_t m3 = __ballot((int32_t)(u3 | 0xFFFFF000u) < Fc);
                            const uint32_t q = (uint32_t)(__mul24(Fc, (int32_t)(z1 >> pvc::PROB_BITS)) + (int32_t)u3);
                            const uint32_t s3 = (ffbh(q) - 8) & 24;
                            const uint32_t q1 = (uint32_t)(((((uint64_t)q << 32) | (uint32_t)(Vc >> 32)) << s3) >> 32);
                            const uint32_t res = q1 | ((s1 + s2 + s3) << 24);          // state | payload bits read
                            uint32_t L;
                            asm volatile("s_ff1_i32_b64 %0, %1" : "=s"(L) : "s"(m1 & m2 & m3));   // -1: no lane
                            const uint32_t pick = rdl(res, L);
                            x = pick & 0xFFFFFF;
                            const uint32_t sb = pick >> 24;
                            V <<= sb; bits += sb;
                            orL |= L; acc = (acc << 6) + L;
                            rr = L;
                        }
                        const uint32_t used = bits >> 3;
                        // a triple with no lane (L = -1), or more bytes than buffered or left in the payload: the sign bits
                        // of the differences (all small), on the scalar unit
                        if ((orL >> 6) | ((d.cnt - used) >> 31) | ((d.n - d.p - used) >> 31)) { stalled = true; break; }
                        d.x = x; d.buf = used < 8 ? d.buf >> (8 * used) : 0; d.cnt -= used; d.p += used; r = rr & 15;
                        if (lane_id() < 3 * G3) blk_put(S, o + j + lane_id(), (uint8_t)(ACGTN >> (8 * ((acc >> (2 * (3 * G3 - 1 - lane_id()))) & 3))));
                        j += 3 * G3;
                    } while (j + 3 * G3 <= (uint32_t)ll);
                    if (!stalled) break;
                    lit.base = o + j;
                    for (uint32_t u = 0; u < 3 * G3; u++, j++) {
                        const uint32_t s = sym_small(d, SR, SR_LIT2 + r);
                        if (d.bad) return -1;
                        uint32_t byte = s < 4 ? (ACGTN >> (8 * s)) & 0xFF : 'N';
                        if (s == 5) { byte = (uint32_t)draw(d, 8); if (d.bad) return -1; }
                        lit.put(S, byte);
                        r = rfl(((r * 4) + (s < 4 ? s : 0)) & 15);
                    }
                    lit.flush(S);
                }
                lit.base = o + j;
                for (; j < (uint32_t)ll; j++) {
                    const uint32_t s = sym_small(d, SR, SR_LIT2 + r);
                    if (d.bad) return -1;
                    uint32_t byte = s < 4 ? (ACGTN >> (8 * s)) & 0xFF : 'N';
                    if (s == 5) { byte = (uint32_t)draw(d, 8); if (d.bad) return -1; }
                    lit.put(S, byte);
                    r = rfl(((r * 4) + (s < 4 ? s : 0)) & 15);
                }
            }
            lit.flush(S);
            o += (uint32_t)ll;
        }
        if (o == blen) break;
        const int kind = (int)sym_small(d, SR, SR_KIND + pvc::llc(ll) * 4 + pvc::kclass(prevk));
        if (d.bad) return -1;
        uint64_t p = 0; uint32_t dir = 0; int ki = 0; int64_t dd = 0; uint64_t dist = 0;
        if (kind == pvc::K_CONT) {
        } else if (kind == pvc::K_DELTA) {
            dd = pvc::unzigzag(dval_big(S, d, BR_DELTA + (ll == 0 ? 0 : 1)));
        } else if (kind == pvc::K_REP) {
            ki = 1 + (int)sym_small(d, SR, SR_REPK);
            if (d.bad) return -1;
            dd = pvc::unzigzag(dval_big(S, d, BR_REPD));
            if ((uint32_t)ki >= C.n) return -1;
        } else if (kind == pvc::K_ABS) {
            dir = sym_small(d, SR, SR_DIR);
            if (d.bad) return -1;
            p = draw(d, 32);
        } else if (kind == pvc::K_SELF) {
            dist = dval_big(S, d, BR_SELF);
        } else if (kind == pvc::K_FLIP) {
            ki = (int)sym_small(d, SR, SR_FLIPK);
            if (d.bad) return -1;
            dd = pvc::unzigzag(dval_big(S, d, BR_FLIPD));
            if ((uint32_t)ki >= C.n) return -1;
        } else {
            return -1;
        }
        if (d.bad) return -1;
        const uint64_t L = dval_big(S, d, BR_LEN + kind) + pvc::MIN_LEN;
        if (d.bad || L > blen - o) return -1;
        uint32_t okind; uint64_t osrc;
        if (kind == pvc::K_SELF) {
            if (dist == 0 || dist > o) return -1;
            okind = 2; osrc = o - dist;
        } else {
            if (kind == pvc::K_FLIP) {
                const int64_t gc = C.cc((uint32_t)ki); const uint32_t gd = C.dd((uint32_t)ki); dir = gd ^ 1;
                const int64_t e = pvc::diag_locus(gc, gd, o) + dd; if (e < 0) return -1; p = (uint64_t)e;
            } else if (kind != pvc::K_ABS) {
                const uint32_t k = kind == pvc::K_REP ? (uint32_t)ki : 0u;
                const int64_t gc = C.cc(k); const uint32_t gd = C.dd(k); dir = gd;
                const int64_t e = pvc::diag_expect(gc, gd, o, L) + dd; if (e < 0) return -1; p = (uint64_t)e;
            }
            if (p > R.n || L > R.n - p) return -1;
            okind = dir ? 3 : 1; osrc = p;
            C.push(pvc::diag_of(dir, p, o, L), dir);
        }
        if (nops >= (int)Cfg<Q>::MAXCOPY) return -1;   // cannot happen: copies are >= 12 bases
        const uint32_t w1v = o | ((uint32_t)L << 15) | (okind << 30);
        if constexpr (Cfg<Q>::REGOPS) op_put(OP, (uint32_t)nops, (uint32_t)osrc, w1v);
        else if (lane_id() == 0) { if constexpr (!G) { S.S->ops[nops][0] = (uint32_t)osrc; S.S->ops[nops][1] = w1v; } }
        nops++;
        o += (uint32_t)L; prevk = kind;
    }
    if (d.bad || d.x != pvc::RANS_L || d.p != d.n) return -1;
    return nops;
}

// ---- light blocks, one lane per (window, block) slot
// A block with a short payload is mostly copies with a few literals: ~40 symbols, each one a dependent chain of a few
// operations. One wave decoding one such block issues ~10 k mostly scalar instructions; here each lane decodes its own
// slot's block with its own rANS state, so a wave decodes 64 blocks for about the instructions of one. The result is
// the block's ops in the format of the wave decoder's op list - copies, plus literal runs as ops of kind 0 whose
// bytes follow in the slot's literal buffer - written to per-slot scratch; windows_kernel then only replays them.
// A slot off the common path (a payload over LIGHT_PAY bytes, more than LOPS ops or LLIT literals) goes to the heavy
// list, whose waves decode it beside the light lanes (below); without the list (a work buffer with no room for it)
// windows_kernel decodes it itself. Every failure condition of the grammar (csrc/refrel3.h:114-160) fails the slot as there: status bit 1,
// nothing written.
constexpr uint32_t SLOT_BYTES = 768, LOPS = 64, LLIT = 192, LIGHT_PAY = 32;
#ifndef PV_LIGHT16
#define PV_LIGHT16 64
#endif
// the light lanes' payload limit: LIGHT_PAY, or at Q = 16384 (where the rest goes to the wave decoder, which takes a
// slot per wave) PV_LIGHT16
template <int Q> constexpr uint32_t light_pay() { return Q == 16384 ? (uint32_t)PV_LIGHT16 : LIGHT_PAY; }
// a payload this long is a long serial chain (a block of mostly literals): the heavy waves take it first
constexpr uint32_t HEAVY_PAY = 512;
constexpr uint32_t SL_OPS = 64, SL_LIT = SL_OPS + LOPS * 8;
           // slot record layout: header, ops, literal bytes
static_assert(SL_LIT + LLIT <= SLOT_BYTES && LOPS <= WAVE && SL_LIT % 16 == 0 && LOPS <= LITE_OPS, "slot record");
// What slot_kernel and light_decode_kernel found for a slot (header word 0):
//  SLOT_DONE    decoded: ops and literals in the slot's record, windows_kernel replays them
//  SLOT_WAVE    windows_kernel decodes the block itself (a heavy slot of a call without a heavy list, or a small
//               call's slot that the light lane spilled)
//  SLOT_FAILED  the block does not decode (status bit 1)
//  SLOT_RANGE   the window lies outside its assembly (status bit 8, reported by the window's first slot)
//  SLOT_SKIP    the window has fewer blocks than slots
//  SLOT_HEAVY   on the heavy list (entry `counts`): a heavy wave of the decode kernel does it whole
enum : uint32_t { SLOT_WAVE = 0, SLOT_DONE = 1, SLOT_FAILED = 2, SLOT_RANGE = 3, SLOT_SKIP = 4, SLOT_HEAVY = 5 };
// Heavy slots of a large call (over SMALL_SLOTS slots) are scheduled by count, not by slot: one wave per slot, as in
// front_kernel, would hold a wave per slot for its lookups. slot_kernel (one lane per slot, ahead of the decode) finds
// every slot's payload length; a slot with a payload over LIGHT_PAY bytes takes an entry of the call's heavy list (one
// atomic per wave and kind): a payload over HEAVY_PAY bytes (a long serial chain) from the list's front, a shorter one
// from its back. heavy_kernel has one wave per heavy area: wave k decodes the list's k-th entry in take order - the
// long ones first, then the short ones - into heavy area k (heavy_decode); windows_kernel replays it from there. Entries past the call's area count, and the slots the light lanes spill (more ops or literals
// than a slot record holds; they follow the long ones at the front), go to spill_kernel's waves, which do each slot
// whole. The list holds every slot of the call, so no heavy slot is left over; a slot's entry index is kept in its
// header (heavy_mark).
// The list and its counters carry the call's epoch (a number the library draws per launch, never reused in the
// process) in their upper 32 bits, so that words left by earlier calls in a reused buffer read as empty and nothing
// is cleared between calls. So do the entries' done words, which windows_kernel checks: a done word of another epoch
// was not written by this call (a slot no heavy wave did; not reached), and the call reports status bit 4.
// The call's control words (epoch << 32 | count): long and short entries (slot_kernel), spilled entries (the light
// lanes). heavy_kernel and spill_kernel take no ticket: their waves' entries follow from their block index, since a
// counter that every wave of a grid bumps at its start costs more than the decodes it hands out.
struct HeavyCtl { uint64_t hbig, hsmall, hspill, pad[5]; };
static_assert(sizeof(HeavyCtl) == 64, "heavy control");
// A heavy area: a record {state, ops}, the copy ops (u32 src, u32 dst | len << 15 | kind << 30 each) and the block with
// its literals in place, written by heavy_kernel's wave k for the heavy list's k-th entry in take order (k below the
// call's area count; in a small call, by front_kernel's heavy wave for slot k) and replayed by windows_kernel. Entries
// past the area count go to spill_kernel, which does them whole.
enum : uint32_t { HEAVY_DONE = 1, HEAVY_FAILED = 2 };
template <int Q> struct Heavy {
    static constexpr uint32_t OPS = 16, BLK = (OPS + 8 * Cfg<Q>::MAXCOPY + 15) & ~15u, BYTES = (BLK + Q + 255) & ~255u;
};
// An entry's done word: the call's epoch, and above it the entry's area (a heavy wave of the decode kernel decoded it
// there), or DONE_WHOLE with the slot's status bits (spill_kernel did the slot whole).
constexpr uint32_t DONE_WHOLE = 0x80000000u;

// A control word's count in this call (0 for a word of an earlier epoch), and an atomic add to it that starts this
// call's count from 0 first where the word still holds an earlier epoch. Device-scope atomics: coherent across the
// XCDs' L2 caches.
__device__ __forceinline__ uint32_t ctl_read(uint64_t* w, uint32_t epoch) {
    const uint64_t v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (uint32_t)(v >> 32) == epoch ? (uint32_t)v : 0u;
}
__device__ __forceinline__ uint32_t ctl_add(uint64_t* w, uint32_t epoch, uint32_t k, int order = __ATOMIC_RELAXED) {
    uint64_t v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // One attempt is enough: only this call's waves change a word of an earlier epoch, and only to this epoch's 0, so
    // if the exchange fails the word already counts for this call.
    if ((uint32_t)(v >> 32) != epoch)
        (void)__hip_atomic_compare_exchange_strong(w, &v, (uint64_t)epoch << 32, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (uint32_t)(order == __ATOMIC_SEQ_CST ? __hip_atomic_fetch_add(w, (uint64_t)k, __ATOMIC_SEQ_CST, __HIP_MEMORY_SCOPE_AGENT)
                                                : __hip_atomic_fetch_add(w, (uint64_t)k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
// The heavy list of a call: capacity, entries, control and areas inside the work buffer.
struct HeavyList { HeavyCtl* ctl; uint64_t* list; uint64_t* done; uint8_t* area; uint32_t cap, acap, nworkers, nlight, epoch; };
// Everything windows_kernel needs of a slot, written by light_decode_kernel as the slot's 64-byte header so that the
// windows kernel starts from one load instead of the chain window -> assembly record -> block table.
struct SlotHdr {
    uint32_t state;
    uint32_t counts;                 // nops | nlit << 8 | block length << 16
    uint32_t part;                   // the window's part of the block: r0 | r1 << 16 (block positions)
    uint32_t row0;                   // row position of block byte r0 (before a reverse complement)
    int64_t stv;                     // start diagonal c << 1 | strand
    uint64_t bst;                    // stream position of the block's first base
    uint64_t payoff;                 // payload offset in the pool
    int64_t low_base;                // the assembly's first case run in the pool
    uint32_t a;                      // assembly
    uint32_t run0;                   // a case run (index within the assembly) at or before the block's first one
    uint32_t plen;                   // payload bytes
    uint32_t low_cnt;                // the assembly's case runs
};
static_assert(sizeof(SlotHdr) == SL_OPS, "slot header");
// A heavy slot's list entry in its header: bits 16-31 in the state word above the state byte, bits 0-15 in the low half
// of `counts` (the op and literal counts of a light slot; the block length stays in the high half)
__device__ __forceinline__ void heavy_mark(SlotHdr& H, uint32_t i) {
    H.state = SLOT_HEAVY | ((i >> 16) << 8);
    H.counts = (H.counts & 0xFFFF0000u) | (i & 0xFFFFu);
}
__device__ __forceinline__ uint32_t heavy_index(const SlotHdr& H) { return ((H.state >> 8) << 16) | (H.counts & 0xFFFFu); }

// A light lane's rANS decoder. At Q <= 4096 the whole payload (at most LIGHT_PAY bytes) and the bytes the refills
// read past its end are loaded into registers when the lane starts, with 16-byte loads issued together, so that no
// refill waits on memory in the middle of the decode (a payload read is an HBM miss: the pool is read once per call).
// At Q = 16384 (payloads of up to 64 bytes) the twenty registers that would take cost more occupancy than the refills
// cost (config 3's batch 0.86 -> 1.08 ms with them), so the refills read the payload there (LDecMem).
template <uint32_t NW> struct LDec {
    uint32_t x, p, n;         // state, payload bytes consumed, payload length
    uint64_t buf;             // the next cnt payload bytes, first in the low byte
    uint32_t cnt;
    bool bad;
    uint32_t E[NW];           // the payload bytes after buf, four per word (zeros past the loaded ones)
};
// four more payload bytes from the register queue
template <uint32_t NW> __device__ __forceinline__ void l_refill(LDec<NW>& d) {
    d.buf |= (uint64_t)d.E[0] << (8 * d.cnt); d.cnt += 4;
#pragma unroll
    for (uint32_t i = 0; i + 1 < NW; i++) d.E[i] = d.E[i + 1];
    d.E[NW - 1] = 0;
}
// the payload at g into the queue (reads past the payload land in the pool's padding), then the initial state: its
// first three bytes
template <uint32_t NW> __device__ __forceinline__ void l_start(LDec<NW>& d, const uint8_t* g, uint32_t plen) {
#pragma unroll
    for (uint32_t k = 0; k < NW / 4; k++) {
        const v4u v = gload16(g + 16 * k);
        d.E[4 * k] = v.x; d.E[4 * k + 1] = v.y; d.E[4 * k + 2] = v.z; d.E[4 * k + 3] = v.w;
    }
    d.n = plen; d.bad = false; d.buf = 0; d.cnt = 0;
    l_refill(d);
    d.x = (uint32_t)(d.buf & 0xFFFFFF); d.buf >>= 24; d.cnt -= 3; d.p = 3;
}
struct LDecMem {
    uint32_t x, p, n;         // state, payload bytes consumed, payload length
    uint64_t buf;             // the next cnt payload bytes, first in the low byte
    uint32_t cnt;
    bool bad;
    const uint8_t* g;         // payload
    uint32_t q;               // payload index of the first byte not in buf
};
__device__ __forceinline__ void l_refill(LDecMem& d) {
    const uintptr_t A = (uintptr_t)(d.g + d.q);
    const uint32_t* w = (const uint32_t*)(A & ~(uintptr_t)3);
    const uint64_t v = ((((uint64_t)w[1]) << 32) | w[0]) >> (8 * (A & 3));
    d.buf |= (v & 0xFFFFFFFFull) << (8 * d.cnt); d.cnt += 4; d.q += 4;
}
__device__ __forceinline__ void l_start(LDecMem& d, const uint8_t* g, uint32_t plen) {
    d.g = g; d.q = 0; d.n = plen; d.bad = false; d.buf = 0; d.cnt = 0;
    l_refill(d);
    d.x = (uint32_t)(d.buf & 0xFFFFFF); d.buf >>= 24; d.cnt -= 3; d.p = 3;
}
template <class LD> __device__ __forceinline__ void l_renorm(LD& d) {
    if (d.x >= pvc::RANS_L) return;
    if (d.cnt < 2) l_refill(d);
    if (d.p >= d.n) { d.bad = true; return; }
    d.x = (d.x << 8) | (uint32_t)(d.buf & 0xFF); d.buf >>= 8; d.cnt--; d.p++;
    if (d.x >= pvc::RANS_L) return;
    if (d.p >= d.n) { d.bad = true; return; }
    d.x = (d.x << 8) | (uint32_t)(d.buf & 0xFF); d.buf >>= 8; d.cnt--; d.p++;
}
// small context: cum[0..7] in one 16-byte load; the symbol is the number of cum[1..6] <= slot
template <class LD> __device__ __forceinline__ uint32_t l_sym_small(LD& d, const uint8_t* tab, uint32_t ctx) {
    const uint4 r = *(const uint4*)(tab + 2 * pvc::row_of((int)ctx));
    const uint32_t slot = d.x & (pvc::M - 1);
    const uint32_t s = (uint32_t)(slot >= (r.x >> 16)) + (uint32_t)(slot >= (r.y & 0xFFFF)) + (uint32_t)(slot >= (r.y >> 16)) +
                       (uint32_t)(slot >= (r.z & 0xFFFF)) + (uint32_t)(slot >= (r.z >> 16)) + (uint32_t)(slot >= (r.w & 0xFFFF));
    const uint64_t X0 = ((uint64_t)r.y << 32) | r.x, X1 = ((uint64_t)r.w << 32) | r.z;
    const uint32_t lo = (uint32_t)((s < 4 ? X0 >> (16 * s) : X1 >> (16 * (s - 4))) & 0xFFFF);
    const uint32_t hi = (uint32_t)((s + 1 < 4 ? X0 >> (16 * (s + 1)) : X1 >> (16 * (s - 3))) & 0xFFFF);
    const uint32_t f = hi - lo;
    if (!f) { d.bad = true; return s; }
    d.x = f * (d.x >> pvc::PROB_BITS) + slot - lo;
    l_renorm(d);
    return s;
}
// big context k (0..14): the slot's bucket entry gives the symbol and its range for a slot among the entry's first three
// symbols (one load); past them, step along the row from the fourth
template <class LD> __device__ __forceinline__ uint32_t l_sym_big(LD& d, const uint8_t* tab, uint32_t k) {
    const uint32_t slot = d.x & (pvc::M - 1);
    const uint64_t e = ((const uint64_t*)(tab + pvc::DIRECT_OFF))[k * pvc::DIRECT_NB + slot / pvc::DIRECT_W];
    const uint32_t s0 = (uint32_t)e & 127, lo0 = (uint32_t)(e >> 7) & 0xFFF;
    const uint32_t e1 = (uint32_t)(e >> 19) & 0xFFF, e2 = (uint32_t)(e >> 31) & 0xFFF, e3 = (uint32_t)(e >> 43) & 0xFFF;
    if (s0 >= (uint32_t)pvc::BIG_ALPHA) { d.bad = true; return 0; }       // an all-zero context
    uint32_t s, lo, f;
    if (slot <= e3) {
        const uint32_t i1 = slot > e1, i2 = slot > e2;
        s = s0 + i1 + i2;
        lo = i2 ? e2 + 1 : i1 ? e1 + 1 : lo0;
        f = (i2 ? e3 : i1 ? e2 : e1) + 1 - lo;
    } else {
        const uint16_t* row = (const uint16_t*)(tab + pvc::SMALL_BYTES) + k * pvc::BIG_ROW;
        s = s0 + 3; lo = e3 + 1;
        uint32_t hi = row[s + 1];
        while (hi <= slot && s < (uint32_t)pvc::BIG_ALPHA - 1) { s++; lo = hi; hi = row[s + 1]; }
        f = hi - lo;
        if (!f || slot < lo) { d.bad = true; return s; }
    }
    d.x = f * (d.x >> pvc::PROB_BITS) + slot - lo;
    l_renorm(d);
    return s;
}
template <class LD> __device__ __forceinline__ uint64_t l_draw(LD& d, uint32_t nb) {
    uint64_t v = 0; uint32_t sh = 0;
    while (nb && !d.bad) {
        const uint32_t k = nb > 16 ? 16 : nb;
        const uint32_t b = d.x & ((1u << k) - 1); d.x >>= k;
        l_renorm(d);
        v |= (uint64_t)b << sh; sh += k; nb -= k;
    }
    return v;
}
template <class LD> __device__ __forceinline__ uint64_t l_dval(LD& d, const uint8_t* tab, uint32_t k) {
    const uint32_t s = l_sym_big(d, tab, k);
    if (d.bad) return 0;
    return pvc::unbucket(s, l_draw(d, pvc::nbits_of(s)));
}
// the block table entry of block b of archive record ar (plain or compact form), one lane at a time
__device__ __forceinline__ void l_block(const pv_dev_cohort& D, const int64_t* ar, uint64_t b, uint64_t bb, uint32_t& poff, uint32_t& plen,
                                        int64_t& stv, int64_t& run0) {
    if (!(D.form & PV_FORM_COMPACT_BLOCKS)) { poff = D.off[bb]; plen = D.off[bb + 1] - poff; stv = D.st[bb]; run0 = D.run0[bb]; return; }
    const uint64_t g = (uint64_t)ar[5] + b / PV_GROUP, first = bb - b % PV_GROUP;
    run0 = D.run0g[g];
    uint64_t o = (uint64_t)D.grp_off[g]; int64_t st = D.grp_st[g];
    for (uint64_t k = first + 1; k <= bb; k++) {
        o += D.blen[k - 1];
        const int32_t c = D.bcode[k];
        if (c == PV_CODE_EXC) {
            int64_t lo = 0, hi = D.nexc;
            while (lo < hi) { const int64_t m = (lo + hi) >> 1; if (D.exc_b[m] < (int64_t)k) lo = m + 1; else hi = m; }
            st = D.exc_st[lo];
        } else {
            const int64_t pc = st >> 1, pred = (st & 1) ? pc - (int64_t)D.Q : pc + (int64_t)D.Q;
            st = (int64_t)(((uint64_t)(pred + (c >> 1)) << 1) | (uint32_t)(c & 1));
        }
    }
    poff = (uint32_t)o; plen = D.blen[bb]; stv = st;
}

// Cohort.sample's coordinates, computed by light_decode_kernel's lanes themselves (one launch fewer per call): the
// window of draw u lies in contig k = the number of entries of the running count cum that are <= u, at u - cum[k-1]
// (the searchsorted / gather / add of the reference's Cohort.sample, panvram/cohort.py:177-189; the same result as
// sample_coords_kernel). draws == nullptr: the windows come from wasm / wstart.
struct SampleIn {
    const int64_t* cum; int64_t nctg; const int64_t* draws; const float* rnd; float p; int rcmode;
    const int64_t* ctg_asm; const int64_t* ctg_local; const int64_t* ctg_boff;
    int64_t* wasm; int64_t* wstart; uint8_t* wrc; int64_t* coords; int* status;
    // a fetch: one window at (fa, fs), strand rcmode, given by value (draws null); slot 0's lane writes them to the
    // call's coordinate record (wasm, wstart, wrc) for the later kernels and zeroes the status word
    int64_t fa, fs; int fixed;
};
// a fetch's record: the window's coordinates, its strand byte and zeros after it, and the status word's zero
__device__ __forceinline__ void fetch_record(const SampleIn& X) {
    X.wasm[0] = X.fa; X.wstart[0] = X.fs;
    *(int64_t*)X.wrc = X.rcmode ? 1 : 0;
    *(int64_t*)X.status = 0;
}
// The count of cum entries <= u is found 16 entries per step: the unknown part [lo, lo + len) is cut into 16 chunks,
// the last entries of all 16 are loaded at once (independent loads, one round trip), the chunks ending at or below u
// are passed over and the first chunk ending above u, less that last entry, stays unknown; four steps for 13,392
// contigs where a binary search takes 14 dependent loads.
__device__ __forceinline__ void lane_coords(const SampleIn& X, uint64_t w, bool writer, int64_t& as, int64_t& st) {
    const int64_t u = X.draws[w];
    int64_t lo = 0, len = X.nctg;
    while (len > 0) {
        const int64_t step = (len + 15) / 16;
        int64_t c = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int64_t a = (int64_t)i * step;
            c += (a < len && X.cum[lo + min(a + step, len) - 1] <= u) ? 1 : 0;
        }
        const int64_t rest = len - c * step;
        lo += min(c * step, len);
        len = rest > 0 ? min(step, rest) - 1 : 0;
    }
    const int64_t k = lo;
    int64_t loc = 0, pos = 0;
    as = -1; st = 0;
    if (k < X.nctg) { pos = u - (k > 0 ? X.cum[k - 1] : 0); as = X.ctg_asm[k]; loc = X.ctg_local[k]; st = X.ctg_boff[k] + pos; }
    if (writer) {
        const uint8_t strand = X.rcmode == 1 ? 1 : (X.rcmode == 2 && X.rnd[w] < X.p) ? 1 : 0;
        X.wasm[w] = as; X.wstart[w] = st;
        if (X.rcmode) X.wrc[w] = strand;
        if (X.coords) { int64_t* co = X.coords + 4 * w; co[0] = as; co[1] = loc; co[2] = pos; co[3] = strand; }
    }
}


// The slot description from the window tables and the block table, when no light_decode_kernel ran before (block size
// 16384, or the light path off): window -> assembly record -> block table entry. Returns false for a slot past the
// window's last block. In the compact-block form the block's group gives its first block's offset, start and case
// run; lane k < nk adds the length of block first + k and lane k in 1..nk turns the code of block first + k into its
// step from the previous block's start (the format's prediction, previous c + Q or - Q by its strand, plus the coded
// difference). The start of b is the last absolute start at or before it (the group's, or an exception's) plus the
// steps after it.
template <int Q>
__device__ __forceinline__ bool slot_at(const pv_dev_cohort& D, int64_t a, int64_t s0, uint32_t W, uint32_t j, SlotHdr& H) {
    const uint32_t l = lane_id();
    H = SlotHdr{};
    H.state = SLOT_RANGE;
    if (a < 0 || a >= D.nasm) return true;
    const int64_t* ar = D.asm_rec + 8 * a;
    const int64_t nbases = ar[2];
    if (s0 < 0 || (uint64_t)s0 + W > (uint64_t)nbases) return true;
    const uint64_t s = (uint64_t)s0;
    const uint64_t b0 = s / Q, b1 = (s + W - 1) / Q, b = b0 + j;
    if (b > b1) return false;
    const uint64_t bst = b * Q;
    const uint32_t blen = (uint32_t)min((uint64_t)Q, (uint64_t)nbases - bst);
    const uint64_t bb = (uint64_t)ar[1] + b;
    uint32_t poff, plen; int64_t stv, run0;
    if (D.form & PV_FORM_COMPACT_BLOCKS) {
        const uint64_t g = (uint64_t)ar[5] + b / PV_GROUP, first = bb - b % PV_GROUP;
        const uint32_t nk = (uint32_t)(b % PV_GROUP);
        const uint32_t len = l < nk ? D.blen[first + l] : 0u;
        const int32_t code = (l >= 1 && l <= nk) ? (int32_t)D.bcode[first + l] : 0;
        const int32_t cprev = __shfl_up(code, 1);
        uint32_t tot = len;
        for (int m = 32; m >= 1; m >>= 1) tot += __shfl_xor(tot, m);
        poff = (uint32_t)D.grp_off[g] + rfl(tot);
        plen = D.blen[bb];
        run0 = D.run0g[g];
        const uint64_t exc = __ballot(code == PV_CODE_EXC);
        uint32_t e = 0; int64_t se = D.grp_st[g];
        if (exc) {
            e = 63u - (uint32_t)__clzll((unsigned long long)exc);
            int64_t lo = 0, hi = D.nexc;                      // the exception entry of pooled block first + e
            const int64_t key = (int64_t)(first + e);
            while (lo < hi) { const int64_t m = (lo + hi) >> 1; if (D.exc_b[m] < key) lo = m + 1; else hi = m; }
            se = D.exc_st[lo];
        }
        const uint32_t dprev = l == e + 1 ? (uint32_t)(se & 1) : (uint32_t)(cprev & 1);
        int32_t step = (l > e && l <= nk) ? (dprev ? -(int32_t)Q : (int32_t)Q) + (code >> 1) : 0;
        for (int m = 32; m >= 1; m >>= 1) step += __shfl_xor(step, m);
        const int64_t c = (se >> 1) + (int64_t)(int32_t)rfl((uint32_t)step);
        const uint32_t dir = nk == e ? (uint32_t)(se & 1) : (uint32_t)(rdl((uint32_t)code, nk) & 1);
        stv = (int64_t)(((uint64_t)c << 1) | dir);
    } else {
        poff = D.off[bb]; plen = D.off[bb + 1] - poff; stv = D.st[bb]; run0 = D.run0[bb];
    }
    const uint32_t r0 = (uint32_t)(max(s, bst) - bst), r1 = (uint32_t)(min(s + W, bst + blen) - bst);
    H.state = SLOT_WAVE; H.counts = blen << 16; H.part = r0 | r1 << 16; H.row0 = (uint32_t)(bst + r0 - s); H.stv = stv; H.bst = bst;
    H.payoff = (uint64_t)ar[0] + poff; H.low_base = ar[3]; H.a = (uint32_t)a; H.run0 = (uint32_t)run0; H.plen = plen;
    H.low_cnt = (uint32_t)ar[4];
    return true;
}
template <int Q>
__device__ __forceinline__ bool slot_from_tables(const pv_dev_cohort& D, const int64_t* wasm, const int64_t* wstart, uint32_t W, uint64_t w,
                                                 uint32_t j, SlotHdr& H) {
    return slot_at<Q>(D, rfl64(wasm[w]), rfl64(wstart[w]), W, j, H);
}

// The draw's contig for a whole wave: the count of cum entries <= u by a 64-way search (the unknown part [lo, lo + len)
// is cut into 64 chunks; lane i tests the last entry of chunk i; the chunks ending at or below u are passed over and
// the first chunk ending above u, less that entry, stays unknown): three rounds for 13,392 contigs.
__device__ __forceinline__ int64_t wave_find(const int64_t* cum, int64_t nctg, int64_t u) {
    const uint32_t l = lane_id();
    int64_t lo = 0, len = nctg;
    while (len > 0) {
        const int64_t step = (len + WAVE - 1) / WAVE;
        const int64_t a = (int64_t)l * step;
        const bool le = a < len && cum[lo + min(a + step, len) - 1] <= u;
        const int64_t c = (int64_t)__popcll(__ballot(le));
        const int64_t rest = len - c * step;
        lo += min(c * step, len);
        len = rest > 0 ? min(step, rest) - 1 : 0;
    }
    return lo;
}

// ---- helpers of the replay's bulk fill (below)

// complement of four bytes (upper-case A <-> T, C <-> G, every other byte unchanged): per byte, 0x80 marks a zero byte of
// w ^ letter (exact, no carries between bytes), then A/T flip by 0x15 and C/G by 0x04
__host__ __device__ __forceinline__ uint32_t comp4(uint32_t w) {
    auto zero = [](uint32_t v) { return ~(((v & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | v) & 0x80808080u; };
    const uint32_t at = zero(w ^ 0x41414141u) | zero(w ^ 0x54545454u), cg = zero(w ^ 0x43434343u) | zero(w ^ 0x47474747u);
    return w ^ ((at >> 7) * 0x15u) ^ ((cg >> 7) * 0x04u);
}
// complement keeping case (pvc::comp_case) of four bytes: the case bit set aside, comp4 on the rest (exact for every
// byte value: only a / c / g / t become A / C / G / T without it)
__host__ __device__ __forceinline__ uint32_t comp_case4(uint32_t w) { return comp4(w & 0xDFDFDFDFu) | (w & 0x20202020u); }
// the token code (pvc::token) of four bytes: b | 0x20 == 'a' / 'c' / 'g' / 't' -> 0 / 1 / 2 / 3, every other byte 4
__host__ __device__ __forceinline__ uint32_t token4(uint32_t w) {
    auto zero = [](uint32_t v) { return ~(((v & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | v) & 0x80808080u; };
    const uint32_t u = w | 0x20202020u;
    const uint32_t za = zero(u ^ 0x61616161u), zc = zero(u ^ 0x63636363u), zg = zero(u ^ 0x67676767u), zt = zero(u ^ 0x74747474u);
    return ((~(za | zc | zg | zt) & 0x80808080u) >> 5) | (zc >> 7) | ((zg >> 7) << 1) | ((zt >> 7) * 3u);
}
// bits 0-3 of b spread to 0x20 in bytes 0-3 (four lower-case flags as the bytes' case bit; the shifted copies of the
// multiplier land on disjoint bits, so no carries)
__host__ __device__ __forceinline__ uint32_t case4(uint32_t b) { return (((b & 0xFu) * 0x00204081u) & 0x01010101u) * 0x20u; }
// 16 bytes at byte offset so of a dword array in LDS (reads five dwords)
__device__ __forceinline__ v4u lds16(const uint32_t* a, uint32_t so) {
    const uint32_t e = so >> 2, sb = so & 3;
    const uint32_t w0 = a[e], w1 = a[e + 1], w2 = a[e + 2], w3 = a[e + 3], w4 = a[e + 4];
    v4u v;
    v.x = __builtin_amdgcn_alignbyte(w1, w0, sb); v.y = __builtin_amdgcn_alignbyte(w2, w1, sb);
    v.z = __builtin_amdgcn_alignbyte(w3, w2, sb); v.w = __builtin_amdgcn_alignbyte(w4, w3, sb);
    return v;
}
// One slot of a window from its decoded or undecoded block to the row (defined below); LS: Lds<Q>, or LdsLite<Q> for the
// replay only (no decode) with a byte reference
template <int Q, bool DEC, class LS>
__device__ __forceinline__ void process_slot(LS& S, const pv_dev_cohort& D, const SlotHdr& H, uint32_t state, const uint8_t* slot_pre,
                                             uint2 op0, const uint8_t* hs, uint32_t hnops, uint64_t w, uint32_t W, bool rc, int tokens,
                                             int apply_case, void* out, const int64_t* ids, int* status);

// The heavy list entry a heavy wave took t-th: slot_kernel's long ones from the front, then its short ones from the back
__device__ __forceinline__ uint32_t entry_at(const HeavyList& HL, uint32_t nbig, uint32_t t) { return t < nbig ? t : HL.cap - 1u - (t - nbig); }

// The window of a heavy list entry's slot, found again from the call's inputs (for sample: the draw, by a 64-way search
// of the running count, and the strand from the uniform draw); slot_kernel put the slot on the list after the same
// lookup on the same inputs.
template <int Q>
__device__ __forceinline__ bool entry_slot(const pv_dev_cohort& D, const int64_t* wasm, const int64_t* wstart, const uint8_t* rcm, uint32_t W,
                                           uint32_t bpw, const SampleIn& X, uint64_t slot, uint64_t& w, bool& rc, SlotHdr& H) {
    w = slot / bpw;
    const uint32_t j = (uint32_t)(slot % bpw);
    int64_t a = -1, s0 = 0;
    if (X.draws) {
        const int64_t u = rfl64(X.draws[w]);
        const int64_t k = rfl64(wave_find(X.cum, X.nctg, u));
        if (k < X.nctg) { a = rfl64(X.ctg_asm[k]); s0 = rfl64(X.ctg_boff[k] + u - (k > 0 ? X.cum[k - 1] : 0)); }
        rc = X.rcmode == 1 || (X.rcmode == 2 && X.rnd[w] < X.p);
    } else if (X.fixed) {
        a = X.fa; s0 = X.fs;
        rc = X.rcmode == 1;
    } else {
        a = rfl64(wasm[w]); s0 = rfl64(wstart[w]);
        rc = rcm && rcm[w];
    }
    return slot_at<Q>(D, a, s0, W, j, H) && rfl(H.state) == SLOT_WAVE;
}

// The wave decoder's decode of a slot's block into heavy area hs, in global memory (no LDS), at raised issue priority
// for a long payload: the record {HEAVY_DONE, ops} or {HEAVY_FAILED, 0}, the copy ops and the block with its literals.
template <int Q>
__device__ __forceinline__ void decode_to_area(const pv_dev_cohort& D, const SlotHdr& H, uint8_t* hs) {
    const uint32_t l = lane_id();
    int nops = -1;
    const uint32_t blen = rfl(H.counts) >> 16, plen = rfl(H.plen);
    const int64_t stv = rfl64(H.stv);
    const uint8_t* gtab = D.tab + (uint64_t)rfl(H.a) * pvc::GTAB_BYTES;
    Small SR;
    {
        const uint4 r = l < (uint32_t)pvc::NSMALL ? ((const uint4*)gtab)[l] : make_uint4(0, 0, 0, 0);
        SR.a = (r.x >> 16) | (r.y << 16); SR.b = (r.y >> 16) | (r.z << 16); SR.c = (r.z >> 16) | (r.w << 16);
    }
    Dec d; d.p = 0; d.n = plen; d.bad = false; d.g = D.P + (uint64_t)rfl64((int64_t)H.payoff);
    d.buf = 0; d.cnt = 0; d.q = 0;
    RefView R; R.g = D.ref; R.n = D.ref_n; R.wbase = 0; R.wlen = 0;
    R.pw = (D.form & PV_FORM_PACKED_REF) ? D.pw : nullptr; R.pes = D.pes; R.pel = D.pel; R.peb = D.peb; R.peix = D.peix; R.pne = D.pne;
    OpRegs<Q> OP;
    OP.src = (v8u)(0u); OP.w1 = (v8u)(0u);
    DecMem<Q, true> M; M.S = nullptr; M.blk = hs + Heavy<Q>::BLK; M.big = (const uint16_t*)(gtab + pvc::SMALL_BYTES);
    // The decoder reads the payload through the scalar cache, four bytes at a time: one miss per 64-byte line,
    // each an HBM round trip on the serial path. One vector load per line (lane i: line i, the first 64 lines),
    // issued first, brings the lines into L2; its value is only consumed at the end, so nothing waits for it.
    // (The pool is padded by 1 KiB past the last payload, which covers the last line.)
    uint32_t sink = 0;
    {
        const uint8_t* p0 = (const uint8_t*)((uintptr_t)d.g & ~(uintptr_t)63);
        const uint32_t nl = (uint32_t)(((uintptr_t)d.g + plen + 8 - (uintptr_t)p0 + 63) / 64);
        typedef const __attribute__((address_space(1))) uint32_t* gptr_t;    // a global (not flat) load: no lgkmcnt
        if (l < nl) sink = *(gptr_t)(uintptr_t)(p0 + 64 * (size_t)l);
    }
    if (plen >= 3) {
        refill(d);
        d.x = (uint32_t)(d.buf & 0xFFFFFF); d.buf >>= 24; d.cnt -= 3; d.p = 3;
        if (plen > HEAVY_PAY) __builtin_amdgcn_s_setprio(3);
        nops = (int)rfl((uint32_t)decode_block(M, OP, d, SR, gtab, R, blen, stv >> 1, (uint32_t)(stv & 1)));
        __builtin_amdgcn_s_setprio(0);
    }
    asm volatile("" ::"v"(sink));
    uint2* ops = (uint2*)(hs + Heavy<Q>::OPS);
#pragma unroll
    for (int r = 0; r < Cfg<Q>::NOPR; r++) {
        const uint32_t k = l + (uint32_t)r * WAVE;
        if ((int)k < nops) ops[k] = make_uint2(OP.src[r], OP.w1[r]);
    }
    *(uint2*)hs = make_uint2(nops >= 0 ? HEAVY_DONE : HEAVY_FAILED, nops >= 0 ? (uint32_t)nops : 0u);   // identical stores
}

// A wave of heavy_kernel: wave k decodes the heavy list's k-th entry in take order (entry_at: the long ones first, then
// the short ones) into heavy area k with the wave decoder, in global memory, at raised issue priority for a long
// payload; the entry's done word then names the area. The grid has one wave per area, so each wave has at most one
// entry: the waves past the list's length (most of them) leave after reading its two counts, and entries past the area
// count are left to spill_kernel. The list is final when the kernel starts (slot_kernel wrote it), so no wave waits.
// Returns the slot it decoded, -1 past the list, -2 for an entry of another call (not reached).
template <int Q>
__device__ __forceinline__ int64_t heavy_decode(const pv_dev_cohort& D, const int64_t* wasm, const int64_t* wstart, uint32_t W, uint32_t bpw,
                                                const SampleIn& X, const HeavyList& HL) {
    const uint32_t nbig = rfl(ctl_read(&HL.ctl->hbig, HL.epoch)), nsmall = rfl(ctl_read(&HL.ctl->hsmall, HL.epoch));
    const uint32_t t = blockIdx.x;
    if (t >= min(nbig + nsmall, HL.acap)) return -1;
    const uint32_t i = entry_at(HL, nbig, t);
    const uint64_t e = (uint64_t)rfl64((int64_t)__hip_atomic_load(&HL.list[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if ((uint32_t)(e >> 32) != HL.epoch) return -2;  // (not reached) windows_kernel reports the slot as status bit 4
    uint64_t w; bool rc; SlotHdr H;
    uint8_t* hs = HL.area + (uint64_t)t * Heavy<Q>::BYTES;
    if (entry_slot<Q>(D, wasm, wstart, nullptr, W, bpw, X, (uint32_t)e, w, rc, H)) decode_to_area<Q>(D, H, hs);
    else *(uint2*)hs = make_uint2(HEAVY_FAILED, 0u);
    HL.done[i] = (uint64_t)HL.epoch | ((uint64_t)t << 32);
    return (int64_t)(uint32_t)e;
}

// A wave of spill_kernel: of the heavy list entries past the call's area count and then the light lanes' spilled ones
// (which follow slot_kernel's long ones at the front), wave k takes items k, k + G, k + 2G, ... (G waves), and does
// each slot whole in its LDS - the wave decoder, the replay, the write-out (process_slot) - then leaves the call's
// epoch, DONE_WHOLE and the slot's status bits in the entry's done word. Both sets are final when the kernel starts.
enum : uint32_t { SPILL_ALL = 0, SPILL_LIST = 1, SPILL_LANES = 2 };
template <int Q>
__device__ __forceinline__ void whole_worker(Lds<Q>& S, const pv_dev_cohort& D, const int64_t* wasm, const int64_t* wstart, const uint8_t* rcm,
                                             uint32_t W, uint32_t bpw, const SampleIn& X, const HeavyList& HL, int tokens, int apply_case,
                                             void* out, const int64_t* ids, int* bits, int* status, uint32_t part) {
    const uint32_t nbig = rfl(ctl_read(&HL.ctl->hbig, HL.epoch)), nsmall = rfl(ctl_read(&HL.ctl->hsmall, HL.epoch));
    const uint32_t over = nbig + nsmall > HL.acap ? nbig + nsmall - HL.acap : 0u;
    // part SPILL_LIST: the list entries past the areas only (slot_kernel's, final before light_decode_kernel runs, so
    // this part may run beside it); SPILL_LANES: the light lanes' spilled ones only; SPILL_ALL: both
    const uint32_t nspill = part == SPILL_LIST ? 0u : rfl(ctl_read(&HL.ctl->hspill, HL.epoch));
    const uint32_t u0 = part == SPILL_LANES ? over : 0u, u1 = part == SPILL_LIST ? over : over + nspill;
    for (uint32_t u = u0 + blockIdx.x; u < u1; u += gridDim.x) {
        const uint32_t i = u < over ? entry_at(HL, nbig, HL.acap + u) : nbig + (u - over);
        const uint64_t e = (uint64_t)rfl64((int64_t)__hip_atomic_load(&HL.list[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if ((uint32_t)(e >> 32) != HL.epoch) {           // (not reached)
            if (lane_id() == 0) atomicOr(status, PV_ST_WAIT);
            continue;
        }
        uint64_t w; bool rc; SlotHdr H;
        *bits = 0;                                     // the slot's status bits, in LDS (process_slot ors into them)
        __syncthreads();
        if (entry_slot<Q>(D, wasm, wstart, rcm, W, bpw, X, (uint32_t)e, w, rc, H))
            process_slot<Q, true>(S, D, H, SLOT_WAVE, nullptr, make_uint2(0, 0), nullptr, 0, w, W, rc, tokens, apply_case, out, ids, bits);
        else
            *bits = PV_ST_DECODE;
        __syncthreads();
        const uint32_t b = rfl((uint32_t)*bits);
        if (b && lane_id() == 0) atomicOr(status, (int)b);
        HL.done[i] = (uint64_t)HL.epoch | ((uint64_t)(DONE_WHOLE | b) << 32);
    }
}

// A slot's header, by its lane: the window (for sample: from the draw; the window's first slot writes its coordinates),
// its block's table entry, the payload length. True for a slot whose payload is over LIGHT_PAY bytes (state SLOT_WAVE);
// a payload under 3 bytes fails the slot.
template <int Q>
__device__ __forceinline__ bool slot_header(const pv_dev_cohort& D, const int64_t* wasm, const int64_t* wstart, uint32_t W, uint32_t bpw,
                                            uint64_t nslots, const SampleIn& X, uint64_t slot, SlotHdr& H) {
    H = SlotHdr{};
    H.state = SLOT_RANGE;
    bool heavy = false;
    if (slot < nslots) do {
        const uint64_t w = slot / bpw; const uint32_t j = (uint32_t)(slot % bpw);
        int64_t a, s0;
        if (X.draws) lane_coords(X, w, j == 0, a, s0);
        else if (X.fixed) { a = X.fa; s0 = X.fs; }
        else { a = wasm[w]; s0 = wstart[w]; }
        if (a < 0 || a >= D.nasm) break;
        const int64_t* ar = D.asm_rec + 8 * a;
        const int64_t nbases = ar[2];
        if (s0 < 0 || (uint64_t)s0 + W > (uint64_t)nbases) break;
        const uint64_t b0 = (uint64_t)s0 / Q, b1 = ((uint64_t)s0 + W - 1) / Q, b = b0 + j;
        H.state = SLOT_SKIP;
        if (b > b1) break;
        const uint64_t bst = b * Q, bb = (uint64_t)ar[1] + b, s = (uint64_t)s0;
        const uint32_t blen = (uint32_t)min((uint64_t)Q, (uint64_t)nbases - bst);
        uint32_t poff, plen; int64_t stv, run0;
        l_block(D, ar, b, bb, poff, plen, stv, run0);
        const uint32_t r0 = (uint32_t)(max(s, bst) - bst), r1 = (uint32_t)(min(s + W, bst + blen) - bst);
        H.counts = blen << 16; H.part = r0 | r1 << 16; H.row0 = (uint32_t)(bst + r0 - s); H.stv = stv; H.bst = bst;
        H.payoff = (uint64_t)ar[0] + poff; H.low_base = ar[3]; H.a = (uint32_t)a; H.run0 = (uint32_t)run0; H.plen = plen;
        H.low_cnt = (uint32_t)ar[4];
        H.state = SLOT_WAVE;
        if (plen > light_pay<Q>()) { heavy = true; break; }
        if (plen < 3) H.state = SLOT_FAILED;
    } while (false);
    return heavy;
}

// The slots' headers, one lane per slot (slot_header); a payload over LIGHT_PAY bytes takes a heavy list entry (long
// ones at the front, the rest at the back).
template <int Q>
__global__ void __launch_bounds__(WAVE) slot_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm, const int64_t* __restrict__ wstart,
                                                    uint32_t W, uint32_t bpw, uint64_t nslots, uint8_t* __restrict__ slotbuf, SampleIn X,
                                                    HeavyList HL) {
    const uint64_t slot = (uint64_t)blockIdx.x * WAVE + threadIdx.x;
    if (X.draws && slot == 0) *X.status = 0;                    // every status bit is set later, by windows_kernel
    if (X.fixed && slot == 0) fetch_record(X);
    const uint32_t lane = lane_id();
    SlotHdr H;
    const bool heavy = slot_header<Q>(D, wasm, wstart, W, bpw, nslots, X, slot, H);
    const bool big = heavy && H.plen > HEAVY_PAY;
    const uint64_t mb = __ballot(big), ms = __ballot(heavy && !big);
    if (HL.cap && (mb | ms)) {
        uint32_t bb = 0, bs = 0;
        if (lane == 0) {
            if (mb) bb = ctl_add(&HL.ctl->hbig, HL.epoch, (uint32_t)__popcll(mb));
            if (ms) bs = ctl_add(&HL.ctl->hsmall, HL.epoch, (uint32_t)__popcll(ms));
        }
        bb = rfl(bb); bs = rfl(bs);
        if (heavy) {
            const uint64_t below = (1ull << lane) - 1ull;
            const uint32_t i = big ? bb + (uint32_t)__popcll(mb & below) : HL.cap - 1u - (bs + (uint32_t)__popcll(ms & below));
            heavy_mark(H, i);
            HL.list[i] = ((uint64_t)HL.epoch << 32) | (uint32_t)slot;
        }
    }
    if (slot < nslots) {
        uint4* hv = (uint4*)(slotbuf + slot * SLOT_BYTES);
        const uint4* hs = (const uint4*)&H;
        hv[0] = hs[0]; hv[1] = hs[1]; hv[2] = hs[2]; hv[3] = hs[3];
    }
}

// A short payload's decode by the slot's lane (H: the slot's header, state SLOT_WAVE, payload of 3 to LIGHT_PAY
// bytes): the block's ops and literal bytes to the slot's record, state SLOT_DONE with the counts, or SLOT_FAILED.
// True when the block needs more ops or literals than a record holds (the header is then unchanged).
// LT: the assembly's model table is in LDS at `ltab` (a one-window call's, staged by its wave), else read from HBM.
template <int Q, bool LT = false>
__device__ __forceinline__ bool light_lane(const pv_dev_cohort& D, uint64_t slot, uint8_t* slotbuf, SlotHdr& H, const uint8_t* ltab = nullptr) {
    bool spilled = false;
    do {
        const uint32_t blen = H.counts >> 16, plen = H.plen;
        const int64_t a = H.a, stv = H.stv;
        const uint8_t* tab = LT ? ltab : D.tab + (uint64_t)a * pvc::GTAB_BYTES;
        RefView R; R.g = D.ref; R.n = D.ref_n; R.wbase = 0; R.wlen = 0;
        R.pw = (D.form & PV_FORM_PACKED_REF) ? D.pw : nullptr; R.pes = D.pes; R.pel = D.pel; R.peb = D.peb; R.peix = D.peix; R.pne = D.pne;
        // at Q <= 4096 the payload and the (at most five) bytes the refills read past its end, in 16-byte loads
        typename std::conditional<Q == 16384, LDecMem, LDec<4 * ((LIGHT_PAY + 5 + 15) / 16)>>::type d;
        l_start(d, D.P + H.payoff, plen);
        uint2* ops = (uint2*)(slotbuf + slot * SLOT_BYTES + SL_OPS);
        uint8_t* lits = slotbuf + slot * SLOT_BYTES + SL_LIT;
        // the four-entry move-to-front diagonal cache (csrc/refrel3.h:94-102), one lane's own
        int64_t cc0 = stv >> 1, cc1 = 0, cc2 = 0, cc3 = 0; uint32_t cd0 = (uint32_t)(stv & 1), cd1 = 0, cd2 = 0, cd3 = 0; int cn = 1;
        int prevk = -1; uint32_t o = 0, nops = 0, nlit = 0;
        bool spill = false;
        // The record is written in 32-byte groups of four ops and 16-byte groups of literal bytes (the partial ones at
        // the end): a store counts in the wave's vector memory counter until it completes, so each store ahead of a
        // table read would hold back the wait for that read.
        uint2 opb0 = make_uint2(0, 0), opb1 = opb0, opb2 = opb0;      // ops nops & ~3 .. nops - 1 (not yet stored)
        uint64_t lacc0 = 0, lacc1 = 0;                                // literal bytes from the 16-byte boundary at or below nlit
        auto put_op = [&](uint2 v) {
            switch (nops & 3) {
                case 0: opb0 = v; break;
                case 1: opb1 = v; break;
                case 2: opb2 = v; break;
                default:
                    *(uint4*)(ops + (nops - 3)) = make_uint4(opb0.x, opb0.y, opb1.x, opb1.y);
                    *(uint4*)(ops + (nops - 1)) = make_uint4(opb2.x, opb2.y, v.x, v.y);
            }
            nops++;
        };
        constexpr uint32_t ACGTN = 'A' | ('C' << 8) | ('G' << 16) | ('T' << 24);
        while (o < blen && !d.bad && !spill) {
            const uint64_t ll = l_dval(d, tab, (uint32_t)pvc::kclass(prevk));
            if (d.bad || ll > blen - o) { d.bad = true; break; }
            if (ll) {
                if (nops >= LOPS || nlit + ll > LLIT) { spill = true; break; }
                put_op(make_uint2(nlit, o | ((uint32_t)ll << 15)));
                // a short run's contexts read the reference bases its diagonal predicts, at most 8 consecutive positions:
                // the 16 bytes from the 8-byte boundary below the lowest one, loaded once (the device reference carries
                // 1 KiB of padding), instead of one dependent load per literal
                uint64_t pre0 = 0, pre1 = 0; int64_t pbase = -1;
                if (ll <= 8 && !R.pw) {
                    const int64_t q0 = pvc::diag_locus(cc0, cd0, o), qb = cd0 ? q0 - (int64_t)ll + 1 : q0;
                    if (qb >= 0 && (uint64_t)qb < R.n) {
                        pbase = qb & ~(int64_t)7;
                        const uint64_t* pp = (const uint64_t*)(R.g + pbase);
                        pre0 = pp[0]; pre1 = pp[1];
                    }
                }
                uint32_t r = 16;
                for (uint32_t k = 0; k < (uint32_t)ll && !d.bad; k++) {
                    uint32_t ctx;
                    if (ll <= 8) {
                        const int64_t q = pvc::diag_locus(cc0, cd0, o + k);
                        uint32_t rb = 4;
                        if (q >= 0 && (uint64_t)q < R.n) {
                            uint32_t byte;
                            if (pbase >= 0) {
                                const uint32_t t = (uint32_t)(q - pbase);          // 0..15: the run lies in the 16 bytes
                                byte = (uint32_t)((t < 8 ? pre0 >> (8 * t) : pre1 >> (8 * (t - 8))) & 0xFF);
                            } else {
                                byte = R.pw ? packed_at(R, (uint64_t)q) : R.g[q];
                            }
                            rb = base_code(byte, cd0);
                        }
                        ctx = pvc::C_LITR + rb * 2 + (k == 0 ? 1 : 0);
                    } else {
                        ctx = pvc::C_LIT2 + r;
                    }
                    const uint32_t sy = l_sym_small(d, tab, ctx);
                    if (d.bad) break;
                    uint32_t byte = sy < 4 ? (ACGTN >> (8 * sy)) & 0xFF : 'N';
                    if (sy == 5) byte = (uint32_t)l_draw(d, 8);
                    const uint32_t q16 = nlit + k;
                    if (q16 & 8) lacc1 |= (uint64_t)(byte & 0xFF) << (8 * (q16 & 7));
                    else lacc0 |= (uint64_t)(byte & 0xFF) << (8 * (q16 & 7));
                    if ((q16 & 15) == 15) {
                        *(uint4*)(lits + (q16 & ~15u)) = make_uint4((uint32_t)lacc0, (uint32_t)(lacc0 >> 32), (uint32_t)lacc1, (uint32_t)(lacc1 >> 32));
                        lacc0 = lacc1 = 0;
                    }
                    r = ((r * 4) + (sy < 4 ? sy : 0)) & 15;
                }
                if (d.bad) break;
                nlit += (uint32_t)ll; o += (uint32_t)ll;
            }
            if (o == blen) break;
            const int kind = (int)l_sym_small(d, tab, pvc::C_KIND + pvc::llc(ll) * 4 + pvc::kclass(prevk));
            if (d.bad || kind > pvc::K_FLIP) { d.bad = true; break; }
            // One decode path for every kind, since the lanes of a wave hold different kinds and a branch per kind would
            // run each kind's decode in turn: the kind's small symbol (REP, FLIP: the cache entry; ABS: the strand), then
            // its value (DELTA, REP, FLIP: the diagonal shift, zigzag coded; SELF: the distance; ABS: 32 raw bits), in
            // the order they were coded (csrc/refrel3.h:136-142)
            uint32_t aux = 0;
            if (kind == pvc::K_REP || kind == pvc::K_FLIP || kind == pvc::K_ABS)
                aux = l_sym_small(d, tab, kind == pvc::K_REP ? pvc::C_REPK : kind == pvc::K_FLIP ? pvc::C_FLIPK : pvc::C_DIR);
            uint64_t val = 0;
            if (!d.bad && kind == pvc::K_ABS) {
                val = l_draw(d, 32);
            } else if (!d.bad && kind != pvc::K_CONT) {
                val = l_dval(d, tab, kind == pvc::K_DELTA ? 4 + (ll == 0 ? 0 : 1) : kind == pvc::K_REP ? 6 : kind == pvc::K_SELF ? 7 : 14);
            }
            if (d.bad) break;
            uint64_t p = 0; uint32_t dir = 0; int ki = 0; int64_t dd = 0; uint64_t dist = 0;
            if (kind == pvc::K_ABS) {
                dir = aux; p = val;
            } else if (kind == pvc::K_SELF) {
                dist = val;
            } else if (kind != pvc::K_CONT) {
                dd = pvc::unzigzag(val);
                ki = kind == pvc::K_REP ? 1 + (int)aux : kind == pvc::K_FLIP ? (int)aux : 0;
                if (ki >= cn) { d.bad = true; break; }
            }
            const uint64_t L = l_dval(d, tab, 8 + (uint32_t)kind) + pvc::MIN_LEN;
            if (d.bad || L > blen - o) { d.bad = true; break; }
            uint32_t okind; uint64_t osrc;
            if (kind == pvc::K_SELF) {
                if (dist == 0 || dist > o) { d.bad = true; break; }
                okind = 2; osrc = o - dist;
            } else {
                const int k = kind == pvc::K_REP ? ki : kind == pvc::K_FLIP ? ki : 0;
                const int64_t gc = k == 0 ? cc0 : k == 1 ? cc1 : k == 2 ? cc2 : cc3;
                const uint32_t gd = k == 0 ? cd0 : k == 1 ? cd1 : k == 2 ? cd2 : cd3;
                if (kind == pvc::K_FLIP) {
                    dir = gd ^ 1;
                    const int64_t e = pvc::diag_locus(gc, gd, o) + dd; if (e < 0) { d.bad = true; break; } p = (uint64_t)e;
                } else if (kind != pvc::K_ABS) {
                    dir = gd;
                    const int64_t e = pvc::diag_expect(gc, gd, o, L) + dd; if (e < 0) { d.bad = true; break; } p = (uint64_t)e;
                }
                if (p > R.n || L > R.n - p) { d.bad = true; break; }
                okind = dir ? 3 : 1; osrc = p;
                // move-to-front push of the copy's diagonal
                const int64_t nc = pvc::diag_of(dir, p, o, L);
                int jx = cn;
                if (cn > 0 && cc0 == nc && cd0 == dir) jx = 0;
                else if (cn > 1 && cc1 == nc && cd1 == dir) jx = 1;
                else if (cn > 2 && cc2 == nc && cd2 == dir) jx = 2;
                else if (cn > 3 && cc3 == nc && cd3 == dir) jx = 3;
                if (jx == cn) { if (cn < 4) cn++; jx = cn - 1; }
                if (jx >= 3) { cc3 = cc2; cd3 = cd2; }
                if (jx >= 2) { cc2 = cc1; cd2 = cd1; }
                if (jx >= 1) { cc1 = cc0; cd1 = cd0; }
                cc0 = nc; cd0 = dir;
            }
            // (at Q = 16384 a self copy goes to the whole-slot pass too: the replay there keeps only the window's part)
            if (nops >= LOPS || (okind == 2 && D.Q == 16384)) { spill = true; break; }
            put_op(make_uint2((uint32_t)osrc, o | ((uint32_t)L << 15) | (okind << 30)));
            o += (uint32_t)L; prevk = kind;
        }
        if (spill) { spilled = true; break; }                   // more ops or literals than a slot record holds
        if (d.bad || d.x != pvc::RANS_L || d.p != d.n) { H.state = SLOT_FAILED; break; }
        if (nops & 3) {
            const uint32_t b = nops & ~3u;
            ops[b] = opb0;
            if ((nops & 3) > 1) ops[b + 1] = opb1;
            if ((nops & 3) > 2) ops[b + 2] = opb2;
        }
        if (nlit & 15)
            *(uint4*)(lits + (nlit & ~15u)) = make_uint4((uint32_t)lacc0, (uint32_t)(lacc0 >> 32), (uint32_t)lacc1, (uint32_t)(lacc1 >> 32));
        H.counts |= nops | nlit << 8;
        H.state = SLOT_DONE;
    } while (false);
    return spilled;
}

// The heavy waves of a large call (heavy_decode), in a kernel of their own: the light lanes then run without the
// wave decoder's registers.
template <int Q>
__global__ void __launch_bounds__(WAVE) heavy_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm, const int64_t* __restrict__ wstart,
                                                     uint32_t W, uint32_t bpw, SampleIn X, HeavyList HL) {
    (void)heavy_decode<Q>(D, wasm, wstart, W, bpw, X, HL);
}

// The decode of the slots slot_kernel left to the light path (SLOT_WAVE with a short payload), one lane per slot.
template <int Q>
__global__ void __launch_bounds__(WAVE) light_decode_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm, const int64_t* __restrict__ wstart,
                                                          uint32_t W, uint32_t bpw, uint64_t nslots, uint8_t* __restrict__ slotbuf,
                                                          SampleIn X, HeavyList HL) {
    const uint64_t slot = (uint64_t)blockIdx.x * WAVE + threadIdx.x;
    const uint32_t lane = lane_id();
    SlotHdr H{};
    bool decodable = false;
    if (slot < nslots) {
        const uint4* hp = (const uint4*)(slotbuf + slot * SLOT_BYTES);
        uint4* hs = (uint4*)&H;
        hs[0] = hp[0]; hs[1] = hp[1]; hs[2] = hp[2]; hs[3] = hp[3];
        decodable = H.state == SLOT_WAVE && H.plen <= light_pay<Q>();
    }
    // Below 16 K block size, a wave whose slots are all of one assembly (a long window's, a stream decode's) stages that
    // model table in LDS first, so that its lanes' table reads wait on LDS instead of L2; a wave of mixed assemblies
    // reads them from HBM. (At 16 K the whole-slot pass runs beside this kernel and needs 50 KB of LDS per wave: the
    // table's 10 KB per wave here would hold it back.)
    bool spilled = false;
    bool staged = false;
    if constexpr (Q != 16384) {
        const uint64_t dm = __ballot(decodable);
        const uint32_t a0 = dm ? rdl(H.a, (uint32_t)__builtin_ctzll(dm)) : 0u;
        if (dm && !__ballot(decodable && H.a != a0)) {
            __shared__ __align__(16) uint8_t tl[pvc::GTAB_BYTES + 16];
            const uint32_t mis = stage(tl, D.tab + (uint64_t)a0 * pvc::GTAB_BYTES, pvc::GTAB_BYTES, pvc::GTAB_BYTES + 16);
            stage_wait();
            if (decodable) spilled = light_lane<Q, true>(D, slot, slotbuf, H, tl + mis);
            staged = true;
        }
    }
    if (!staged && decodable) spilled = light_lane<Q>(D, slot, slotbuf, H);
    // a spilled slot takes an entry after slot_kernel's long ones (one atomic per wave)
    const uint64_t m = __ballot(spilled);
    if (m && HL.cap) {
        uint32_t base = 0;
        if (lane == 0) base = ctl_add(&HL.ctl->hspill, HL.epoch, (uint32_t)__popcll(m));
        base = rfl(base) + rfl(ctl_read(&HL.ctl->hbig, HL.epoch));
        if (spilled) {
            const uint32_t i = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
            heavy_mark(H, i);
            __hip_atomic_store(&HL.list[i], ((uint64_t)HL.epoch << 32) | (uint32_t)slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (decodable) *(uint2*)(slotbuf + slot * SLOT_BYTES) = make_uint2(H.state, H.counts);   // windows_kernel sets the status bits
}

// Calls of at most SMALL_SLOTS slots take one kernel before windows_kernel, which keeps a short call's latency to its
// longest serial decode. Its first HL.nworkers waves (one per slot, or none without a heavy list) are the heavy role: a
// slot whose payload is over LIGHT_PAY bytes is decoded by its wave into heavy area `slot` (decode_to_area), which
// done word `slot` then names; every other slot's wave exits after its lookup. The light waves follow, one lane per
// slot: the header (slot_header) and a short payload's decode (light_lane); a heavy slot's header points at done word
// `slot` (the heavy role found it by the same lookup on the same inputs), and a spilled slot stays SLOT_WAVE for
// windows_kernel's wave decoder.
constexpr uint64_t SMALL_SLOTS = 16384;
// At Q = 16384 the other path's replay holds less LDS (the window's part of the block) and its whole-slot passes run
// beside the replay: it takes calls of more than 2,048 slots (sample(1024, 65536): 3.13 -> 5.03 M windows/s; 32768:
// 5.60 -> 6.51 M; 4,096 fetches: 4.15 -> 6.06 M; at 256 slots sample(1024, 1024) lost 14 %).
constexpr uint64_t SMALL_SLOTS_Q16 = 2048;
template <int Q> constexpr uint64_t small_slots() { return Cfg<Q>::REGOPS ? SMALL_SLOTS : SMALL_SLOTS_Q16; }
// ONE: a call of one window of at most 64 slots (a fetch): its light wave stages the window's assembly's model table in
// LDS (every slot shares it) before its lanes decode, so that the decode's table reads wait on LDS, not on L2 or HBM.
template <int Q, bool ONE = false>
__global__ void __launch_bounds__(WAVE) front_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm, const int64_t* __restrict__ wstart,
                                                     uint32_t W, uint32_t bpw, uint64_t nslots, uint8_t* __restrict__ slotbuf, SampleIn X,
                                                     HeavyList HL) {
    if constexpr (Cfg<Q>::REGOPS) {                   // (no heavy role where ops live in LDS: nworkers is 0)
        if (blockIdx.x < HL.nworkers) {
            const uint64_t slot = blockIdx.x;
            uint64_t w; bool rc; SlotHdr H;
            if (!entry_slot<Q>(D, wasm, wstart, nullptr, W, bpw, X, slot, w, rc, H) || rfl(H.plen) <= light_pay<Q>()) return;
            decode_to_area<Q>(D, H, HL.area + slot * Heavy<Q>::BYTES);
            HL.done[slot] = (uint64_t)HL.epoch | (slot << 32);
            return;
        }
    }
    const uint64_t slot = (uint64_t)(blockIdx.x - HL.nworkers) * WAVE + threadIdx.x;
    if (X.draws && slot == 0) *X.status = 0;                    // every status bit is set later, by windows_kernel
    if (X.fixed && slot == 0) fetch_record(X);
    SlotHdr H;
    const bool heavy = slot_header<Q>(D, wasm, wstart, W, bpw, nslots, X, slot, H);
    if (heavy) { if (HL.nworkers) heavy_mark(H, (uint32_t)slot); }
    if constexpr (ONE) {
        __shared__ __align__(16) uint8_t tl[pvc::GTAB_BYTES + 16];
        const uint64_t m = __ballot(!heavy && H.state == SLOT_WAVE);
        if (m) {                                   // (wave-uniform) the slots' assembly, from the first lane to decode
            const uint32_t a = rdl(H.a, (uint32_t)__builtin_ctzll(m));
            const uint32_t mis = stage(tl, D.tab + (uint64_t)a * pvc::GTAB_BYTES, pvc::GTAB_BYTES, pvc::GTAB_BYTES + 16);
            stage_wait();
            if (!heavy && H.state == SLOT_WAVE) (void)light_lane<Q, true>(D, slot, slotbuf, H, tl + mis);
        }
    } else {
        if (!heavy && H.state == SLOT_WAVE) (void)light_lane<Q>(D, slot, slotbuf, H);
    }
    if (slot < nslots) {
        uint4* hv = (uint4*)(slotbuf + slot * SLOT_BYTES);
        const uint4* hs = (const uint4*)&H;
        hv[0] = hs[0]; hv[1] = hs[1]; hv[2] = hs[2]; hv[3] = hs[3];
    }
}

// After the decode kernels, the slots the heavy areas did not take and the light lanes' spilled ones (both rare in
// cohorts of long haplotypes: more heavy slots than areas, a short payload with more ops or literals than a slot record
// holds), each whole by a wave of their own as far as the grid goes: one wave per 16 slots, at least one per heavy area.
// A cohort whose long blocks are common (a tenth of them or more) spills most of them: its calls then take one whole
// slot per wave or two instead of a queue of them; where nothing spills the waves leave after reading three counts.
constexpr uint32_t SPILL_SLOTS = 16;
inline uint32_t spill_waves(uint64_t nslots, uint32_t areas) {
    const uint64_t w = (nslots + SPILL_SLOTS - 1) / SPILL_SLOTS;
    return (uint32_t)(w > areas ? w : areas);
}
template <int Q>
__global__ void __launch_bounds__(WAVE) spill_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm, const int64_t* __restrict__ wstart,
                                                   uint32_t W, uint32_t bpw, SampleIn X, HeavyList HL, const uint8_t* __restrict__ rcm,
                                                   int tokens, int apply_case, void* __restrict__ out, const int64_t* __restrict__ ids,
                                                   int* __restrict__ status, uint32_t part) {
    __shared__ Lds<Q> S;
    __shared__ int bits;
    whole_worker<Q>(S, D, wasm, wstart, rcm, W, bpw, X, HL, tokens, apply_case, out, ids, &bits, status, part);
}

// One slot of a window: the block's replay into the wave's LDS `S`, after a decode there where the block arrives
// undecoded (DEC, state SLOT_WAVE), then the write-out of the window's part of it with the transforms (lower case,
// reverse complement, tokens or ids). H: the slot's header; slot_pre: its record (ops and literal bytes of a light
// slot); op0: lane l's op of the record's first 16; hs, hnops: the heavy area of a slot a heavy wave decoded (state
// SLOT_HEAVY) and its copy op count. Failures set status bits.
template <int Q, bool DEC, class LS>
__device__ __forceinline__ void process_slot(LS& S, const pv_dev_cohort& D, const SlotHdr& H, uint32_t state, const uint8_t* slot_pre,
                                             uint2 op0, const uint8_t* hs, uint32_t hnops, uint64_t w, uint32_t W, bool rc, int tokens,
                                             int apply_case, void* out, const int64_t* ids, int* status) {
    constexpr bool SPAN = LS::SPAN;           // false: no staged reference span, no literal bytes in LDS (HBM / L2 reads)
    constexpr bool WINB = LS::WIN;            // blk / lower start at block position xb (a multiple of 32)
    static_assert(SPAN || !DEC, "the wave decoder needs the staged span");
    const uint32_t l = lane_id();
    // Every value a branch below takes is read as wave-uniform (one lane's copy; all lanes hold the same), so that
    // each early return leaves with the whole wave: this function also runs inside a heavy wave's loop over slots.
    state = rfl(state); rc = rfl(rc ? 1u : 0u) != 0;
    const bool light = state == SLOT_DONE, wave = state == SLOT_WAVE, heavy = state == SLOT_HEAVY;
    hnops = rfl(hnops);
    const uint32_t counts = rfl(H.counts), part = rfl(H.part);
    const uint32_t blen = counts >> 16, plen = rfl(H.plen);
    const uint32_t r0 = part & 0xFFFF, r1 = part >> 16;            // the window's part of the block
    const uint32_t xb = WINB ? (r0 & ~31u) : 0u;
    const uint64_t bst = (uint64_t)rfl64((int64_t)H.bst);
    const int64_t boff = (int64_t)rfl(H.row0) - (int64_t)r0;       // row position of block byte 0
    const int64_t low_base = rfl64(H.low_base), low_cnt = rfl(H.low_cnt), run0 = rfl(H.run0);
    const int64_t stv = rfl64(H.stv);
    const int64_t g0c = stv >> 1; const uint32_t g0d = (uint32_t)(stv & 1);
    const uint8_t* gpay = D.P + (uint64_t)rfl64((int64_t)H.payoff);
    const uint8_t* gtab = D.tab + (uint64_t)rfl(H.a) * pvc::GTAB_BYTES;

    // A block decoded here reads its payload through the scalar cache, four bytes at a time: one miss per 64-byte
    // line, each an HBM round trip on the serial path. One vector load per line (lane i: line i, the first 64 lines),
    // issued first, brings the lines into L2; its value is only consumed at the end, so nothing waits for it. (The pool
    // is padded by 1 KiB past the last payload, which covers the last line.)
    uint32_t sink = 0;
    if (DEC && wave) {
        const uint8_t* p0 = (const uint8_t*)((uintptr_t)gpay & ~(uintptr_t)63);
        const uint32_t nl = (uint32_t)(((uintptr_t)gpay + plen + 8 - (uintptr_t)p0 + 63) / 64);
        typedef const __attribute__((address_space(1))) uint32_t* gptr_t;    // a global (not flat) load: no lgkmcnt
        if (l < nl) sink = *(gptr_t)(uintptr_t)(p0 + 64 * (size_t)l);
    }

    // 1. model rows, payload windows, reference span (a decoded light slot needs only the span)
    Small SR;
    Dec d; d.p = 0; d.n = plen; d.bad = false; d.g = gpay;
    d.buf = 0; d.cnt = 0; d.q = 0;
    if (wave) {
        const uint4 r = l < (uint32_t)pvc::NSMALL ? ((const uint4*)gtab)[l] : make_uint4(0, 0, 0, 0);
        SR.a = (r.x >> 16) | (r.y << 16); SR.b = (r.y >> 16) | (r.z << 16); SR.c = (r.z >> 16) | (r.w << 16);
    } else {
        SR.a = SR.b = SR.c = 0;
    }
    RefView R; R.g = D.ref; R.n = D.ref_n; R.wbase = 0; R.wlen = 0;
    const bool packed = D.form & PV_FORM_PACKED_REF;
    R.pw = packed ? D.pw : nullptr; R.pes = D.pes; R.pel = D.pel; R.peb = D.peb; R.peix = D.peix; R.pne = D.pne;
    int64_t wl = 0, wh = 0; uint32_t pmis = 0, pwords = 0;
    if constexpr (SPAN) {
        // the start diagonal's image of the block positions needed: the whole block to decode one, the window's part
        // [r0, r1) for a decoded light slot (its copies rarely leave the diagonal by more than the margin; a source
        // outside the staged span is read from HBM)
        const uint32_t x0 = light ? r0 : 0u, x1 = light ? r1 : blen;
        const int64_t lo = g0d ? g0c - (int64_t)x1 + 1 : g0c + (int64_t)x0, hi = lo + (int64_t)(x1 - x0);   // span [lo, hi)
        wl = lo - (int64_t)RMARGIN; wh = hi + (int64_t)RMARGIN;
        if (wl < 0) wl = 0;
        if (wh > (int64_t)D.ref_n) wh = (int64_t)D.ref_n;
        if (wl < wh && !packed) {
            const uint32_t mis = stage<STREAM>(S.refw, D.ref + wl, (uint32_t)(wh - wl), Cfg<Q>::REFW);
            R.wbase = wl - (int64_t)mis;
            R.wlen = min((uint32_t)(wh - wl) + mis, (uint32_t)Cfg<Q>::REFW);
        } else if (wl < wh) {
            // the 2-bit words of the span go to the block buffer (free until the decode; the payload area for a slot
            // whose block arrives decoded) and are unpacked below
            const uint64_t w0 = (uint64_t)wl >> 4;
            pwords = (uint32_t)((((uint64_t)wh + 15) >> 4) - w0);
            pmis = heavy ? stage<STREAM>(S.aux, (const uint8_t*)(D.pw + w0), pwords * 4, Cfg<Q>::AUX)
                         : stage<STREAM>(S.blk, (const uint8_t*)(D.pw + w0), pwords * 4, Q);
            R.wbase = (int64_t)(w0 << 4);
            R.wlen = min(pwords * 16, (uint32_t)Cfg<Q>::REFW);
        }
    }
    // a block decoded here: the rows of its 104-letter contexts, one read per symbol of those contexts (LDS instead of
    // an L2 round trip on the serial path)
    uint32_t bmis = 0;
    if constexpr (DEC) if (wave && plen >= 3) bmis = stage(S.aux, gtab + pvc::SMALL_BYTES, Cfg<Q>::BIG_ROWS, Cfg<Q>::AUX);
    // a decoded light slot: its ops past the first 16 and its literal bytes (to the payload area, unused here) travel
    // with the span
    uint2 opl = op0;
    const uint32_t lnops = light ? (counts & 0xFF) : 0u, lnlit = light ? ((counts >> 8) & 0xFF) : 0u;
    if (light) {
        if (lnops > 16 && l >= 16 && l < lnops) opl = ((const uint2*)(slot_pre + SL_OPS))[l];
        if constexpr (SPAN) { if (lnlit) stage(S.aux, slot_pre + SL_LIT, lnlit, Cfg<Q>::AUX); }
    }
    const uint8_t* glit = light ? slot_pre + SL_LIT : nullptr;      // a light slot's literal bytes in its record
    // a heavy slot: the decoded block to the block buffer, its copy ops to the op registers
    OpRegs<Q> OP;
    OP.src = (v8u)(0u); OP.w1 = (v8u)(0u);
    if constexpr (Cfg<Q>::REGOPS) {
        if (heavy) {
            stage(S.blk, hs + Heavy<Q>::BLK, blen, Q);
            const uint2* hops = (const uint2*)(hs + Heavy<Q>::OPS);
#pragma unroll
            for (int r = 0; r < Cfg<Q>::NOPR; r++) {
                const uint32_t k = l + (uint32_t)r * WAVE;
                if (k < hnops) { const uint2 e = hops[k]; OP.src[r] = e.x; OP.w1[r] = e.y; }
            }
        }
    }
    stage_wait();
    if constexpr (SPAN) if (pwords) {
        // word j -> 16 bytes: each byte of the word holds four 2-bit codes, spread to one code per byte and turned into
        // letters by a byte permute of "ACGT"
        const uint32_t nw = min(pwords, (uint32_t)Cfg<Q>::REFW / 16);
        for (uint32_t j = l; j < nw; j += WAVE) {
            uint32_t wd;
            memcpy(&wd, (heavy ? S.aux : S.blk) + pmis + 4 * j, 4);
            uint4 o;
            uint32_t* op = &o.x;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t x = (wd >> (8 * i)) & 0xFF;
                const uint32_t sel = (x | (x << 6) | (x << 12) | (x << 18)) & 0x03030303u;
                op[i] = __builtin_amdgcn_perm(0u, ACGT, sel);
            }
            *(uint4*)(S.refw + 16 * j) = o;
        }
        __syncthreads();
        // runs of other bytes inside the staged span overwrite their positions
        const uint64_t s0 = (uint64_t)R.wbase, s1 = s0 + R.wlen;
        for (int64_t r = rfl(D.peix[s0 >> PV_EXC_BUCKET_BITS]); r < D.pne; r++) {
            const uint64_t rs = (uint64_t)D.pes[r], re = rs + (uint64_t)D.pel[r];
            if (rs >= s1) break;
            const uint64_t a0 = max(rs, s0), a1 = min(re, s1);
            const uint8_t byte = D.peb[r];
            for (uint64_t q = a0 + l; q < a1; q += WAVE) S.refw[q - s0] = byte;
        }
        __syncthreads();
    }

    // 2. decode
    int nops = -1;
    if (heavy) {
        nops = (int)hnops;
    } else if (light) {
        // at most LOPS (= one per lane) ops, literal runs included
        nops = (int)lnops;
        OP.src[0] = l < lnops ? opl.x : 0u; OP.w1[0] = l < lnops ? opl.y : 0u;
        if constexpr (!Cfg<Q>::REGOPS) { if (l < lnops) { S.ops[l][0] = opl.x; S.ops[l][1] = opl.y; } }
    } else if constexpr (DEC) if (plen >= 3) {
        refill(d);
        d.x = (uint32_t)(d.buf & 0xFFFFFF); d.buf >>= 24; d.cnt -= 3; d.p = 3;
        // a long payload is a long serial chain that bounds its launch: its wave issues ahead of the short-lived ones
        if (plen > HEAVY_PAY) __builtin_amdgcn_s_setprio(3);
        DecMem<Q, false> M; M.S = &S; M.blk = nullptr; M.big = (const uint16_t*)(S.aux + bmis);
        nops = (int)rfl((uint32_t)decode_block(M, OP, d, SR, gtab, R, blen, g0c, g0d));
        __builtin_amdgcn_s_setprio(0);
    }
    asm volatile("" ::"v"(sink));
    if (nops < 0) { atomicOr(status, PV_ST_DECODE); return; }      // (every lane: one atomic after folding)
    __syncthreads();

    // 3. replay the copies the window part [r0, r1) of this block needs
    const bool do_case = apply_case && !tokens && low_cnt > 0;
    uint32_t need = r0;           // lowest block position still needed: self copies pull it down
    auto op_src = [&](int k) -> uint32_t {
        if constexpr (Cfg<Q>::REGOPS) return op_get(OP.src, (uint32_t)k); else return S.ops[k][0];
    };
    auto op_w1 = [&](int k) -> uint32_t {
        if constexpr (Cfg<Q>::REGOPS) return op_get(OP.w1, (uint32_t)k); else return S.ops[k][1];
    };
    // one op's bytes [i0, i1) into the block, all lanes (kind 0: the light slot's literal bytes; 1: reference; 3: reverse
    // complement; 2: the block itself, overlap allowed)
    auto copy_op = [&](uint32_t src, uint32_t w1, uint32_t i0, uint32_t i1) {
        const uint32_t dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF, kind = w1 >> 30;
        // source offset in the staged span (kind 1); a source that starts below the span wraps to a huge value, so the
        // test is on `so` first and on the remaining room after it (no sum that could wrap back into range)
        const uint64_t so = (uint64_t)src + i0 - (uint64_t)R.wbase;
        if constexpr (!SPAN) {
            if (kind == 1 && i1 > i0 + 8) {
                // from HBM: 16 bytes per lane per pass, the destination's first 16-byte boundary splitting the head off
                const uint32_t a0 = dst + i0, a1 = dst + i1, b0 = min((a0 + 15) & ~15u, a1);
                if (l < b0 - a0) S.blk[a0 + l] = ref_at(S, R, (uint64_t)src + i0 + l);
                for (uint32_t q = b0 + 16 * l; q < a1; q += 16 * WAVE) {
                    const uint64_t sq = (uint64_t)src + (q - dst);
                    if (q + 16 <= a1 && sq + 16 <= R.n) {
                        *(v4u*)&S.blk[q] = gload16(R.g + sq);
                    } else {
                        for (uint32_t i = 0; i < 16 && q + i < a1; i++) S.blk[q + i] = ref_at(S, R, sq + i);
                    }
                }
                return;
            }
        } else {
            if (kind == 1 && i1 > i0 + 8 && so < R.wlen && i1 - i0 <= R.wlen - so) {
                // wholly inside the staged span: aligned destination words, each assembled from two source words
                const uint32_t a0 = dst + i0, a1 = dst + i1, b0 = (a0 + 3) & ~3u, b1 = a1 & ~3u;
                const uint32_t sh = (uint32_t)(so + (b0 - a0));      // source offset of destination byte b0
                if (l < b0 - a0) S.blk[a0 + l] = S.refw[so + l];
                if (l < a1 - b1) S.blk[b1 + l] = S.refw[so + (b1 - a0) + l];
                const uint32_t* rw = (const uint32_t*)S.refw;
                for (uint32_t q = b0 + 4 * l; q < b1; q += 4 * WAVE) {
                    const uint32_t o = sh + (q - b0);
                    *(uint32_t*)&S.blk[q] = __builtin_amdgcn_alignbyte(rw[(o >> 2) + 1], rw[o >> 2], o & 3);
                }
                return;
            }
        }
        if (kind == 1) {
            // four bytes per lane in flight per pass
            uint32_t i = i0 + l;
            for (; i + 3 * WAVE < i1; i += 4 * WAVE) {
                const uint8_t v0 = ref_at(S, R, (uint64_t)src + i), v1 = ref_at(S, R, (uint64_t)src + i + WAVE);
                const uint8_t v2 = ref_at(S, R, (uint64_t)src + i + 2 * WAVE), v3 = ref_at(S, R, (uint64_t)src + i + 3 * WAVE);
                S.blk[dst + i] = v0; S.blk[dst + i + WAVE] = v1; S.blk[dst + i + 2 * WAVE] = v2; S.blk[dst + i + 3 * WAVE] = v3;
            }
            for (; i < i1; i += WAVE) S.blk[dst + i] = ref_at(S, R, (uint64_t)src + i);
        } else if (kind == 3) {
            const uint64_t top = (uint64_t)src + len - 1;
            uint32_t i = i0 + l;
            for (; i + 3 * WAVE < i1; i += 4 * WAVE) {
                const uint8_t v0 = ref_at(S, R, top - i), v1 = ref_at(S, R, top - i - WAVE);
                const uint8_t v2 = ref_at(S, R, top - i - 2 * WAVE), v3 = ref_at(S, R, top - i - 3 * WAVE);
                S.blk[dst + i] = pvc::comp(v0); S.blk[dst + i + WAVE] = pvc::comp(v1);
                S.blk[dst + i + 2 * WAVE] = pvc::comp(v2); S.blk[dst + i + 3 * WAVE] = pvc::comp(v3);
            }
            for (; i < i1; i += WAVE) S.blk[dst + i] = pvc::comp(ref_at(S, R, top - i));
        } else if (kind == 0) {
            // a literal run decoded by light_decode_kernel: its bytes, staged from the slot's literal buffer (or read
            // from it)
            if constexpr (SPAN) { for (uint32_t i = i0 + l; i < i1; i += WAVE) S.blk[dst + i] = S.aux[src + i]; }
            else { for (uint32_t i = i0 + l; i < i1; i += WAVE) S.blk[dst + i] = glit[src + i]; }
        } else {
            const uint32_t dist = dst - src;
            for (uint32_t i = i0 + l; i < i1; i += WAVE) S.blk[dst + i] = S.blk[src + (i % dist)];
        }
    };
    // A light block mostly follows its start diagonal (copies on it, with single literals between them for SNVs): fill
    // the needed range along that diagonal from the staged span first, 16 bytes per lane, so that only the ops that
    // leave it are replayed. Only where the diagonal's source for the range (and 16 bytes either side) is in the span.
    auto bulk_fill = [&](uint32_t from) -> bool {
        const int64_t lo = g0d ? g0c - (int64_t)r1 + 1 : g0c + (int64_t)from, hi = g0d ? g0c - (int64_t)from + 1 : g0c + (int64_t)r1;
        if constexpr (SPAN) { if (!(lo - 16 >= R.wbase && hi + 20 <= R.wbase + (int64_t)R.wlen)) return false; }
        else { if (!(lo - 16 >= 0 && hi + 20 <= (int64_t)R.n)) return false; }
        const uint32_t c_hi = (r1 + 15) / 16;
        constexpr uint32_t NCH = (Q / 16 + WAVE - 1) / WAVE;      // chunks per lane at most (the loop's bound when
        const uint32_t c0 = from / 16 + l;                        // Q > 4096)
        auto src16 = [&](int64_t q) -> v4u {                      // reference bytes [q, q + 16)
            if constexpr (SPAN) return lds16((const uint32_t*)S.refw, (uint32_t)(q - R.wbase));
            else return gload16(R.g + q);
        };
        auto chunk = [&](uint32_t c) {
            const uint32_t x = 16 * c;
            v4u v;
            if (!g0d) {
                v = src16(g0c + x);
            } else {
                const v4u u = src16(g0c - (int64_t)x - 15);
                v.x = comp4(__builtin_bswap32(u.w)); v.y = comp4(__builtin_bswap32(u.z));
                v.z = comp4(__builtin_bswap32(u.y)); v.w = comp4(__builtin_bswap32(u.x));
            }
            *(v4u*)&S.blk[x] = v;
        };
        if constexpr (NCH <= 4) {
#pragma unroll
            for (uint32_t k = 0; k < NCH; k++) if (c0 + k * WAVE < c_hi) chunk(c0 + k * WAVE);
        } else {
            for (uint32_t c = c0; c < c_hi; c += WAVE) chunk(c);
        }
        __syncthreads();
        return true;
    };
    auto on_diag = [&](uint32_t src, uint32_t w1) -> bool {
        const uint32_t dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF, kind = w1 >> 30;
        return (kind == 1 && !g0d && (int64_t)src == g0c + (int64_t)dst) || (kind == 3 && g0d && (int64_t)src + (int64_t)len - 1 == g0c - (int64_t)dst);
    };
    // bytes [off, off + 16) of a copy or literal op, from LDS: the literal bytes (kind 0) or the staged span, read forward
    // (kind 1) or backward and complemented (kind 3). False when the span does not hold them all.
    auto op16 = [&](uint32_t src, uint32_t len, uint32_t kind, uint32_t off, v4u& v) -> bool {
        if constexpr (!SPAN) {
            // from the slot record's literal bytes or the reference in HBM (a 16-byte read inside the record or the
            // reference; else false and byte by byte)
            if (kind == 0) {
                if (src + off + 16 > LLIT) return false;
                v = gload16(glit + src + off);
                return true;
            }
            uint64_t q;
            if (kind == 1) {
                q = (uint64_t)src + off;
                if (q + 16 > R.n) return false;
            } else {
                const uint64_t top = (uint64_t)src + len - 1;
                if (top < (uint64_t)off + 15) return false;
                q = top - off - 15;
            }
            const v4u u = gload16(R.g + q);
            if (kind == 1) { v = u; return true; }
            v.x = comp4(__builtin_bswap32(u.w)); v.y = comp4(__builtin_bswap32(u.z));
            v.z = comp4(__builtin_bswap32(u.y)); v.w = comp4(__builtin_bswap32(u.x));
            return true;
        } else {
            if (kind == 0) { v = lds16((const uint32_t*)S.aux, src + off); return true; }
            if (kind == 1) {
                const uint64_t so = (uint64_t)src + off - (uint64_t)R.wbase;
                if (!(so < R.wlen && R.wlen - so >= 20)) return false;
                v = lds16((const uint32_t*)S.refw, (uint32_t)so);
                return true;
            }
            const uint64_t top = (uint64_t)src + len - 1;
            if (top < (uint64_t)off + 15) return false;
            const uint64_t so = top - off - 15 - (uint64_t)R.wbase;
            if (!(so < R.wlen && R.wlen - so >= 20)) return false;
            const v4u u = lds16((const uint32_t*)S.refw, (uint32_t)so);
            v.x = comp4(__builtin_bswap32(u.w)); v.y = comp4(__builtin_bswap32(u.z));
            v.z = comp4(__builtin_bswap32(u.y)); v.w = comp4(__builtin_bswap32(u.x));
            return true;
        }
    };
    // byte off of an op, from wherever its source is (the span, HBM or the literal bytes)
    auto op_byte = [&](uint32_t src, uint32_t len, uint32_t kind, uint32_t off) -> uint8_t {
        if constexpr (SPAN) { if (kind == 0) return S.aux[src + off]; }
        else { if (kind == 0) return glit[src + off]; }
        if (kind == 1) return ref_at(S, R, (uint64_t)src + off);
        return pvc::comp(ref_at(S, R, (uint64_t)src + len - 1 - off));
    };
    bool replayed = false;
    {
        // A light slot without self copies: its <= 64 ops, one per lane, cover the block in order. Every 16-byte chunk
        // of the window part takes 16 bytes of the op that covers its first byte (one copy from LDS); then the lane of
        // each op that starts inside a chunk writes that op's bytes up to the chunk's end over them.
        if (light) {
            const uint32_t w1l = OP.w1[0], srcl = OP.src[0], dl = w1l & 0x7FFF, ll = (w1l >> 15) & 0x7FFF, kl = w1l >> 30;
            const bool mine = l < (uint32_t)nops;
            if (!__ballot(mine && kl == 2)) {
                constexpr uint32_t NCH = ((WINB ? WIN_BYTES : (uint32_t)Q) / 16 + WAVE - 1) / WAVE;      // chunks per lane
                const uint32_t cA = r0 / 16, cB = (r1 + 15) / 16;
                // covering op of chunk c: the last op starting at or before its first byte - k0 for chunk cA, plus the
                // ops after k0 (and before chunk cB) that start at or before it
                const uint32_t k0 = (uint32_t)__popcll(__ballot(mine && dl <= 16 * cA)) - 1u;
                const uint32_t k1 = (uint32_t)__popcll(__ballot(mine && dl < 16 * cB));
                // chunk rounds this window part needs (the part can be much shorter than the buffer): the rounds past
                // it are skipped whole
                const uint32_t nj = rfl((cB - cA + WAVE - 1) / WAVE);
                uint32_t own[NCH];
#pragma unroll
                for (uint32_t j = 0; j < NCH; j++) own[j] = k0;
                for (uint32_t k = k0 + 1; k < k1; k++) {
                    const uint32_t dk = rdl(dl, k);
#pragma unroll
                    for (uint32_t j = 0; j < NCH; j++) if (j < nj) own[j] += 16 * (cA + l + j * WAVE) >= dk ? 1u : 0u;
                }
                // the op-start patch below (the bytes of this lane's op in the chunk where it starts): at !SPAN its
                // 16-byte read is issued here, with the chunks' first reads, and written after the chunks
                const bool patch = mine && (dl & 15) && dl >= 16 * cA && dl < r1;
                bool pok = false;
                v4u pv = {0, 0, 0, 0};
                if constexpr (!SPAN) {
                    const uint8_t* pa = R.g;
                    if (patch) {
                        if (kl == 0) { pok = srcl + 16 <= LLIT; pa = glit + srcl; }
                        else if (kl == 1) { pok = (uint64_t)srcl + 16 <= R.n; pa = R.g + srcl; }
                        else { const uint64_t top = (uint64_t)srcl + ll - 1; pok = top >= 15; pa = R.g + (top - 15); }
                    }
                    pv = gload16(pok ? pa : R.g);
                }
                if constexpr (!SPAN && NCH <= 4) {
                    // from HBM (the reference, or the slot record's literal bytes): the 16-byte reads of all (up to
                    // four) rounds issued before the first is waited for (one round trip per slot, not per round); a
                    // chunk past the part, or whose bytes a 16-byte read cannot take, reads the reference's first
                    // bytes instead and is written byte by byte after. (At q16k, eight or sixteen rounds: the registers
                    // of four in flight cost more workgroups per CU than the round trips they save.)
                    constexpr uint32_t G = NCH;
                    for (uint32_t j0 = 0; j0 < nj; j0 += G) {
                        const uint8_t* ap[G]; uint32_t aw[G], as_[G], ao[G]; bool ok[G];
#pragma unroll
                        for (uint32_t g = 0; g < G; g++) {
                            const uint32_t j = j0 + g, c = cA + l + j * WAVE;
                            const uint32_t oj = own[j < NCH ? j : 0];
                            const uint32_t w1 = (uint32_t)__shfl((int)w1l, (int)oj), src = (uint32_t)__shfl((int)srcl, (int)oj);
                            const uint32_t dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF, kind = w1 >> 30, off = 16 * c - dst;
                            const uint8_t* a = R.g;
                            bool good = false;
                            if (j < nj && c < cB) {
                                if (kind == 0) {
                                    good = src + off + 16 <= LLIT; a = glit + src + off;
                                } else if (kind == 1) {
                                    good = (uint64_t)src + off + 16 <= R.n; a = R.g + (uint64_t)src + off;
                                } else {
                                    const uint64_t top = (uint64_t)src + len - 1;
                                    good = top >= (uint64_t)off + 15; a = R.g + (top - off - 15);
                                }
                            }
                            ap[g] = good ? a : R.g; ok[g] = good; aw[g] = w1; as_[g] = src; ao[g] = off;
                        }
                        v4u vv[G];
#pragma unroll
                        for (uint32_t g = 0; g < G; g++) vv[g] = gload16(ap[g]);
#pragma unroll
                        for (uint32_t g = 0; g < G; g++) {
                            const uint32_t j = j0 + g, c = cA + l + j * WAVE, x0 = 16 * c;
                            if (j < nj && c < cB) {
                                const uint32_t w1 = aw[g], len = (w1 >> 15) & 0x7FFF, kind = w1 >> 30, off = ao[g];
                                if (ok[g]) {
                                    v4u v = vv[g];
                                    if (kind == 3) {
                                        const v4u u = v;
                                        v.x = comp4(__builtin_bswap32(u.w)); v.y = comp4(__builtin_bswap32(u.z));
                                        v.z = comp4(__builtin_bswap32(u.y)); v.w = comp4(__builtin_bswap32(u.x));
                                    }
                                    *(v4u*)&S.blk[x0 - xb] = v;
                                } else {
                                    const uint32_t nb = min(16u, len - off);
                                    for (uint32_t i = 0; i < nb; i++) S.blk[x0 - xb + i] = op_byte(as_[g], len, kind, off + i);
                                }
                            }
                        }
                    }
                } else {
#pragma unroll
                for (uint32_t j = 0; j < NCH; j++) {
                    if (j >= nj) break;
                    const uint32_t c = cA + l + j * WAVE, x0 = 16 * c;
                    const uint32_t w1 = (uint32_t)__shfl((int)w1l, (int)own[j]), src = (uint32_t)__shfl((int)srcl, (int)own[j]);
                    if (c < cB) {
                        const uint32_t dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF, kind = w1 >> 30, off = x0 - dst;
                        v4u v;
                        if (op16(src, len, kind, off, v)) {
                            *(v4u*)&S.blk[x0 - xb] = v;
                        } else {
                            const uint32_t nb = min(16u, len - off);
                            for (uint32_t i = 0; i < nb; i++) S.blk[x0 - xb + i] = op_byte(src, len, kind, off + i);
                        }
                    }
                }
                }
                __syncthreads();
                if (patch) {
                    const uint32_t nb = min(ll, 16 - (dl & 15));          // the op's bytes in its first chunk
                    v4u v = pv;
                    if (!SPAN && pok && kl == 3) {
                        v.x = comp4(__builtin_bswap32(pv.w)); v.y = comp4(__builtin_bswap32(pv.z));
                        v.z = comp4(__builtin_bswap32(pv.y)); v.w = comp4(__builtin_bswap32(pv.x));
                    }
                    if (SPAN ? op16(srcl, ll, kl, 0, v) : pok) {
                        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (uint32_t i = 0; i < 15; i++)
                            if (i < nb) S.blk[dl - xb + i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
                    } else {
                        for (uint32_t i = 0; i < nb; i++) S.blk[dl - xb + i] = op_byte(srcl, ll, kl, i);
                    }
                }
                __syncthreads();
                replayed = true;
            }
        }
    }
    if constexpr (WINB) {
        if (!replayed) { if (l == 0) atomicOr(status, PV_ST_WAIT); return; }     // (not reached: no self copies here)
    } else if (!replayed) {
        int klast = nops - 1;
        while (klast >= 0 && (op_w1(klast) & 0x7FFF) >= r1) klast--;
        int kfirst = klast + 1;
        for (int k = klast; k >= 0; k--) {
            const uint32_t w1 = op_w1(k), dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF;
            if (dst + len <= need) break;     // ops are in block order: every earlier one ends before `need` too
            kfirst = k;
            if ((w1 >> 30) == 2) { const uint32_t src = op_src(k); if (src < need) need = src; }
        }
        const bool bulk = light && bulk_fill(need);
        // Ops write disjoint ranges and read the staged span, the literal bytes or HBM, except self copies, which read
        // the block: a barrier before each of those and one before the write-out.
        for (int k = kfirst; k <= klast; k++) {
            const uint32_t src = op_src(k), w1 = op_w1(k), dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF, kind = w1 >> 30;
            if (bulk && on_diag(src, w1)) continue;
            if (kind == 2) __syncthreads();
            copy_op(src, w1, need > dst ? need - dst : 0, min(len, r1 - dst));
        }
        __syncthreads();
    }

    // 4. lower-case bitmask of [r0, r1), then the write-out with the transforms
    if (do_case) {
        constexpr uint32_t NWORDS = (WINB ? WIN_BYTES : (uint32_t)Q) / 32;   // bitmask words at most, from word xb / 32
        constexpr int NW = (int)((NWORDS + WAVE - 1) / WAVE);
        const uint32_t wd0 = r0 / 32, wd1 = (r1 + 31) / 32, wbase = xb / 32;
        const uint32_t nwd = wd1 - wbase;               // words the write-out reads: [0, nwd) of the bitmask
        uint32_t acc[NW];
        for (int k = 0; k < NW; k++) acc[k] = 0;
        const int64_t* ls = D.low_s + low_base; const int64_t* ln = D.low_l + low_base;
        const uint64_t x0 = bst + r0, x1 = bst + r1;
        for (int64_t r = run0; r < low_cnt; r += WAVE) {
            const int64_t rr = r + l;
            int64_t rs = INT64_MAX, re = INT64_MAX;
            if (rr < low_cnt) { rs = ls[rr]; re = rs + ln[rr]; }
            // runs are sorted: stop once one starts at or after the window part's end
            const uint64_t stop = __ballot(rr < low_cnt && (uint64_t)rs >= x1);
            const uint64_t live = __ballot(rr < low_cnt && (uint64_t)rs < x1 && (uint64_t)re > x0);
            for (uint64_t m = live; m; m &= m - 1) {
                const uint32_t src_l = (uint32_t)(__ffsll((unsigned long long)m) - 1);
                const int64_t a0 = rdl64(rs, src_l), a1 = rdl64(re, src_l);
                const uint32_t q0 = (uint32_t)(max((uint64_t)a0, x0) - bst), q1 = (uint32_t)(min((uint64_t)a1, x1) - bst);
                for (int k = 0; k < NW; k++) {
                    if ((uint32_t)k * WAVE >= nwd) break;
                    const uint32_t wd = wbase + l + (uint32_t)k * WAVE, wb0 = wd * 32, wb1 = wb0 + 32;
                    if (wd < wd0 || wd >= wd1) continue;
                    const uint32_t lo = max(q0, wb0), hi = min(q1, wb1);
                    if (lo < hi) {
                        const uint32_t nbit = hi - lo;
                        acc[k] |= (nbit == 32 ? 0xFFFFFFFFu : ((1u << nbit) - 1)) << (lo - wb0);
                    }
                }
            }
            if (stop) break;
        }
        uint32_t* lower = lower_of(S, W);
        for (int k = 0; k < NW; k++) { const uint32_t wd = l + (uint32_t)k * WAVE; if (wd < nwd) lower[wd] = acc[k]; }
        __syncthreads();
    }
    if (ids) {
        // token ids straight into the caller's int64 rows (the id map of a training loader fused into the store)
        const int64_t i0 = ids[0], i1 = ids[1], i2 = ids[2], i3 = ids[3], i4 = ids[4];
        int64_t* row = (int64_t*)out + w * (uint64_t)W;
        for (uint32_t x = r0 + l; x < r1; x += WAVE) {
            uint8_t v = S.blk[x - xb];
            const uint64_t t = (uint64_t)((int64_t)x + boff);
            uint64_t pos = t;
            if (rc) { v = pvc::comp_case(v); pos = (uint64_t)W - 1 - t; }
            const uint32_t tk = pvc::token(v);
            row[pos] = tk == 0 ? i0 : tk == 1 ? i1 : tk == 2 ? i2 : tk == 3 ? i3 : i4;
        }
        return;
    }
    // The slot's bytes cover row positions [p0, p1) (mirrored for a reverse complement); each lane stores 4-byte
    // aligned words of that range, the unaligned ends go byte by byte.
    uint8_t* row = (uint8_t*)out + w * (uint64_t)W;
    const uint64_t t0 = (uint64_t)((int64_t)r0 + boff), t1 = (uint64_t)((int64_t)r1 + boff);
    const uint64_t p0 = rc ? (uint64_t)W - t1 : t0, p1 = rc ? (uint64_t)W - t0 : t1;
    if (!rc && !tokens && !do_case) {
        // the bytes as they are: 16-byte aligned row chunks, each assembled from five block words
        const uint32_t xo = r0 - xb;                              // buffer position of row byte p0
        const uint64_t head = min(p1 - p0, (uint64_t)((16 - ((uintptr_t)(row + p0) & 15)) & 15));
        if (l < head) row[p0 + l] = S.blk[xo + l];
        const uint64_t pb = p0 + head, nch = (p1 - pb) / 16;
        const uint32_t* bw = (const uint32_t*)S.blk;
        for (uint64_t k = l; k < nch; k += WAVE) {
            const uint32_t x = xo + (uint32_t)(pb - p0) + 16 * (uint32_t)k, e = x >> 2, sb = x & 3;
            const uint32_t w0 = bw[e], w1 = bw[e + 1], w2 = bw[e + 2], w3 = bw[e + 3], w4 = bw[e + 4];
            uint4 v;
            v.x = __builtin_amdgcn_alignbyte(w1, w0, sb); v.y = __builtin_amdgcn_alignbyte(w2, w1, sb);
            v.z = __builtin_amdgcn_alignbyte(w3, w2, sb); v.w = __builtin_amdgcn_alignbyte(w4, w3, sb);
            const v4u nv = {v.x, v.y, v.z, v.w};
            __builtin_nontemporal_store(nv, (v4u*)(row + pb + 16 * k));      // output rows are not read back here
        }
        const uint64_t pt = pb + 16 * nch;
        if (l < p1 - pt) row[pt + l] = S.blk[xo + (uint32_t)(pt - p0) + l];
        return;
    }
    auto byte_at = [&](uint64_t p) -> uint32_t {
        const uint32_t x = (uint32_t)((int64_t)(rc ? (uint64_t)W - 1 - p : p) - boff) - xb;   // (xb: a multiple of 32)
        uint8_t v = S.blk[x];
        if (do_case && ((lower_of(S, W)[x >> 5] >> (x & 31)) & 1)) v |= 0x20;
        if (rc) v = pvc::comp_case(v);
        if (tokens) v = pvc::token(v);
        return v;
    };
    // 16-byte aligned row chunks: the 16 block bytes a chunk shows (read forward; for a reverse complement the chunk's
    // last row byte is the lowest block byte), their 16 lower-case flags as case bits, then the complement and the byte
    // order reversal, then the token codes, four bytes at a time; the unaligned ends byte by byte
    const uint64_t head = min(p1 - p0, (uint64_t)((16 - ((uintptr_t)(row + p0) & 15)) & 15));
    if (l < head) row[p0 + l] = (uint8_t)byte_at(p0 + l);
    const uint64_t pb = p0 + head, nch = (p1 - pb) / 16;
    const uint32_t* bw = (const uint32_t*)S.blk;
    for (uint64_t k = l; k < nch; k += WAVE) {
        const uint64_t p = pb + 16 * k;
        const uint32_t x = (uint32_t)((int64_t)(rc ? (uint64_t)W - 16 - p : p) - boff) - xb;   // lowest buffer position
        const uint32_t e = x >> 2, sb = x & 3;
        const uint32_t w0 = bw[e], w1 = bw[e + 1], w2 = bw[e + 2], w3 = bw[e + 3], w4 = bw[e + 4];
        uint32_t v[4] = {__builtin_amdgcn_alignbyte(w1, w0, sb), __builtin_amdgcn_alignbyte(w2, w1, sb),
                         __builtin_amdgcn_alignbyte(w3, w2, sb), __builtin_amdgcn_alignbyte(w4, w3, sb)};
        if (do_case) {
            const uint32_t wi = x >> 5, sh = x & 31;
            const uint32_t* lower = lower_of(S, W);
            uint64_t lw = lower[wi];
            if (sh > 16) lw |= (uint64_t)lower[wi + 1] << 32;
            const uint32_t bits = (uint32_t)(lw >> sh);
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] |= case4(bits >> (4 * i));
        }
        if (rc) {
            const uint32_t r0w = comp_case4(v[0]), r1w = comp_case4(v[1]), r2w = comp_case4(v[2]), r3w = comp_case4(v[3]);
            v[0] = __builtin_bswap32(r3w); v[1] = __builtin_bswap32(r2w); v[2] = __builtin_bswap32(r1w); v[3] = __builtin_bswap32(r0w);
        }
        if (tokens) {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = token4(v[i]);
        }
        const v4u nv = {v[0], v[1], v[2], v[3]};
        __builtin_nontemporal_store(nv, (v4u*)(row + p));
    }
    const uint64_t pt = pb + 16 * nch;
    if (l < p1 - pt) row[pt + l] = (uint8_t)byte_at(pt + l);
}


// Slot sb of a call: its header (the slot record, or the window and block tables), then the slot by process_slot.
// skip_heavy: a slot on the heavy list is left to heavy_replay_fused_kernel and spill_kernel.
template <int Q, bool DEC, class LS>
__device__ __forceinline__ void window_slot(LS& S, const pv_dev_cohort& D, const int64_t* wasm, const int64_t* wstart, uint32_t W, uint32_t bpw,
                                            const uint8_t* rcm, int tokens, int apply_case, void* out, const int64_t* ids, int* status,
                                            const uint8_t* pre, const uint64_t* hdone, const uint8_t* harea, uint32_t epoch, uint32_t sb,
                                            bool skip_heavy) {
    const uint32_t l = lane_id();
    const uint64_t w = sb / bpw; const uint32_t j = sb % bpw;
    const bool rc = rcm && rcm[w];
    SlotHdr H;
    uint2 op0 = make_uint2(0, 0);                      // a decoded light slot's op `l`, for l < 16
    const uint8_t* slot_pre = pre ? pre + (uint64_t)sb * SLOT_BYTES : nullptr;
    if (slot_pre) {
        // the slot's header and its first 16 ops in one round trip
        const uint4* hp = (const uint4*)slot_pre;
        uint4 hv[4] = {hp[0], hp[1], hp[2], hp[3]};
        if (l < 16) op0 = ((const uint2*)(slot_pre + SL_OPS))[l];
        uint32_t* hw = &hv[0].x;
#pragma unroll
        for (int k = 0; k < 16; k++) hw[k] = rfl(hw[k]);
        memcpy(&H, hv, sizeof(H));
    } else if (!slot_from_tables<Q>(D, wasm, wstart, W, w, j, H)) {
        return;
    }
    uint32_t state = H.state & 0xFF;
    if (state == SLOT_SKIP) return;
    if (state == SLOT_RANGE) { if (l == 0 && j == 0) atomicOr(status, PV_ST_RANGE); return; }
    if (state == SLOT_FAILED) { if (l == 0) atomicOr(status, PV_ST_DECODE); return; }
    const uint8_t* hs = nullptr;
    uint32_t hnops = 0;
    if (state == SLOT_HEAVY) {
        // on the heavy list: its done word names the heavy area the decode kernel decoded it to, or says spill_kernel did
        // the slot whole (it reports the slot's status bits itself); a word of another epoch was not written by this
        // call. Where there are no heavy areas (Q = 16384) spill_kernel does every such slot and may run beside this
        // kernel: the slot is left to it unread.
        if constexpr (!Cfg<Q>::REGOPS) return;
        if (skip_heavy) return;
        const uint64_t done = hdone[heavy_index(H)];
        const uint32_t tag = rfl((uint32_t)(done >> 32));
        if (rfl((uint32_t)done) != epoch) { if (l == 0) atomicOr(status, PV_ST_WAIT); return; }
        if (tag & DONE_WHOLE) return;
        hs = harea + (uint64_t)tag * Heavy<Q>::BYTES;
        const uint2 rec = *(const uint2*)hs;
        hnops = rfl(rec.y);
        if (rfl(rec.x) != HEAVY_DONE || hnops > Cfg<Q>::MAXCOPY) { if (l == 0) atomicOr(status, PV_ST_DECODE); return; }
    } else if (!DEC && state != SLOT_DONE) {
        if (l == 0) atomicOr(status, PV_ST_WAIT);       // (not reached)
        return;
    }
    if constexpr (DEC && LS::SPAN) {
        // a light slot (decoded by its lane: ops and literal bytes in its record) needs no decoder: it replays as in
        // the replay-only kernel, its reads straight from HBM and issued together, without staging the reference span
        // in LDS first (the block's LDS taken as the smaller layout). Not in the packed-reference form, which holds no
        // byte reference to read from: there the span is staged and unpacked.
        if (state == SLOT_DONE && slot_pre && !(D.form & PV_FORM_PACKED_REF)) {
            process_slot<Q, false>(*reinterpret_cast<LdsLite<Q>*>(&S), D, H, state, slot_pre, op0, hs, hnops, w, W, rc, tokens, apply_case,
                                   out, ids, status);
            return;
        }
    }
    process_slot<Q, DEC>(S, D, H, state, slot_pre, op0, hs, hnops, w, W, rc, tokens, apply_case, out, ids, status);
}

template <int Q, bool DEC, bool LITE = false, bool WINDOW = false>
__global__ void __launch_bounds__(WAVE) windows_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm, const int64_t* __restrict__ wstart,
                                                     uint32_t W, uint32_t bpw, const uint8_t* __restrict__ rcm, int tokens, int apply_case,
                                                     void* __restrict__ out, const int64_t* __restrict__ ids, int* __restrict__ status,
                                                     const uint8_t* __restrict__ pre, const uint64_t* __restrict__ hdone,
                                                     const uint8_t* __restrict__ harea, uint32_t xshift, uint32_t epoch, uint32_t skip_heavy) {
    static_assert(!(DEC && LITE) && (LITE || !WINDOW), "the wave decoder needs the staged span; the window buffer is the replay's");
    // Workgroups go to the 8 XCDs round-robin (workgroup b to XCD b % 8). The decode kernels write slot s's record
    // from a workgroup on XCD (xshift + s / 64) % 8 (xshift = 0: slot_kernel's and light_decode_kernel's wave s / 64;
    // front_kernel's light wave comes after its heavy waves); slot s is taken here by a workgroup on that same XCD, so that the record is read
    // through the XCD's own L2. In whole groups of 512 slots, a bijection; the last partial group and xshift = ~0u keep
    // slot = workgroup.
    uint32_t sb = blockIdx.x;
    if (xshift != ~0u && sb < (gridDim.x & ~511u)) {
        const uint32_t m = sb >> 3, x = ((sb & 7) - xshift) & 7;
        sb = ((m >> 6) << 9) | (x << 6) | (m & 63);
    }
    if constexpr (WINDOW) {
        // the window buffer in dynamic LDS: the launch passes offsetof(blk) + win_bytes(W) + the bitmask's bytes
        extern __shared__ __align__(16) uint8_t pv_window_lds[];
        auto& S = *reinterpret_cast<LdsLite<Q, true>*>(pv_window_lds);
        window_slot<Q, DEC>(S, D, wasm, wstart, W, bpw, rcm, tokens, apply_case, out, ids, status, pre, hdone, harea, epoch, sb, skip_heavy != 0);
    } else {
        __shared__ typename std::conditional<LITE, LdsLite<Q>, Lds<Q>>::type S;
        window_slot<Q, DEC>(S, D, wasm, wstart, W, bpw, rcm, tokens, apply_case, out, ids, status, pre, hdone, harea, epoch, sb, skip_heavy != 0);
    }
}

// heavy_kernel's waves, each then replaying the slot it decoded into its output row, after a windows_kernel that left
// the heavy list's slots (skip_heavy): a short heavy slot's replay runs beside the longest blocks' serial chains instead
// of after them, and a long one follows its own chain only. The wave's own stores of the area and the done word are
// visible to its loads after the workgroup fence. LITE: the replay reads the reference from HBM (the byte form), else
// it stages the span.
template <int Q, bool LITE>
__global__ void __launch_bounds__(WAVE) heavy_replay_fused_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm,
                                                                  const int64_t* __restrict__ wstart, uint32_t W, uint32_t bpw, SampleIn X,
                                                                  HeavyList HL, const uint8_t* __restrict__ rcm, int tokens, int apply_case,
                                                                  void* __restrict__ out, const int64_t* __restrict__ ids,
                                                                  int* __restrict__ status, const uint8_t* __restrict__ pre) {
    const int64_t slot = heavy_decode<Q>(D, wasm, wstart, W, bpw, X, HL);
    if (slot < 0) { if (slot == -2 && lane_id() == 0) atomicOr(status, PV_ST_WAIT); return; }
    __threadfence_block();
    __syncthreads();
    __shared__ typename std::conditional<LITE, LdsLite<Q>, Lds<Q>>::type S;
    window_slot<Q, false>(S, D, wasm, wstart, W, bpw, rcm, tokens, apply_case, out, ids, status, pre, (const uint64_t*)HL.done,
                          (const uint8_t*)HL.area, HL.epoch, (uint32_t)slot, false);
}

void seterr(char* e, size_t cap, const char* m) { if (e && cap) snprintf(e, cap, "%s", m); }

// Window coordinates of a sample draw, one wave per window. `cum` is the per-W running count of valid window starts
// over the cohort's contigs (contig k holds cum[k] - cum[k-1] of them); draw u falls in contig k = the number of
// entries with cum <= u. 64-way search: the unknown part of the table is [lo, lo + len); lane i tests the last entry of
// the i-th of 64 equal chunks of it; the c chunks that end at or below u are passed over, and chunk c minus its last
// entry (known to be above u) is what stays unknown - three levels for 13,392 contigs. The window starts at
// u - cum[k-1] in contig k. Also the strand (rnd[i] < p in float32, as torch compares a float tensor with a Python
// float; every window or none for rcmode 1 / 0) and the zeroed status word. A draw past the table gives assembly -1,
// which the decode kernel reports as status bit 8. (What the reference's Cohort.sample computes with torch ops after
// the same two draws, panvram/cohort.py:177-189.)
__global__ void __launch_bounds__(256) sample_coords_kernel(const int64_t* __restrict__ cum, int64_t nctg, const int64_t* __restrict__ draws,
                                                            const float* __restrict__ rnd, float p, int rcmode,
                                                            const int64_t* __restrict__ ctg_asm, const int64_t* __restrict__ ctg_local,
                                                            const int64_t* __restrict__ ctg_boff, int64_t n, int64_t* __restrict__ wasm,
                                                            int64_t* __restrict__ wstart, uint8_t* __restrict__ wrc,
                                                            int64_t* __restrict__ coords, int* __restrict__ status) {
    const uint32_t l = threadIdx.x & (WAVE - 1);
    const int64_t w = (int64_t)blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (w == 0 && l == 0) *status = 0;
    if (w >= n) return;
    const int64_t u = draws[w];
    int64_t lo = 0, len = nctg;
    while (len > 0) {
        const int64_t step = (len + WAVE - 1) / WAVE;
        const int64_t a = (int64_t)l * step;                                   // chunk start, relative to lo
        const bool le = a < len && cum[lo + min(a + step, len) - 1] <= u;
        const int64_t c = (int64_t)__popcll(__ballot(le));
        const int64_t rest = len - c * step;                                   // entries from chunk c on
        lo += min(c * step, len);
        len = rest > 0 ? min(step, rest) - 1 : 0;
    }
    const int64_t k = lo;
    int64_t as = -1, loc = 0, pos = 0, st = 0;
    if (k < nctg) {
        pos = u - (k > 0 ? cum[k - 1] : 0);
        as = ctg_asm[k]; loc = ctg_local[k]; st = ctg_boff[k] + pos;
    }
    const uint8_t strand = rcmode == 1 ? 1 : (rcmode == 2 && rnd[w] < p) ? 1 : 0;
    if (l == 0) {
        wasm[w] = as; wstart[w] = st;
        if (rcmode) wrc[w] = strand;
        if (coords) { int64_t* co = coords + 4 * w; co[0] = as; co[1] = loc; co[2] = pos; co[3] = strand; }
    }
}

// A large call's heavy waves run on a second stream beside its light lanes: per launch stream (per device) a side
// stream and two events, made on the first large call on that stream and kept for the process (at most MAXFORKS
// launch streams per device; past that, and for callers that must not create streams, the two kernels run one after
// the other on the launch stream). The side stream waits for slot_kernel (the heavy list), and the launch stream waits
// for the heavy waves before spill_kernel.
#ifndef PV_FORK
#define PV_FORK 1
#endif
#ifndef PV_LITE
#define PV_LITE 1
#endif
constexpr int MAXFORKS = 64;
struct Fork { hipStream_t st, side, side2; hipEvent_t fork, join, lanes, join2; };
std::mutex fork_mu;
std::vector<Fork> fork_set[64];
// The side stream(s) and events of caller stream st, made on first use: the second side stream (two = true, for the
// whole-slot passes at Q = 16384) only where asked for, since every stream takes one of the process's hardware queues.
// nullptr when they cannot be had (the call then runs on st alone).
const Fork* fork_of(hipStream_t st, bool two = false) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) { (void)hipGetLastError(); return nullptr; }
    std::lock_guard<std::mutex> g(fork_mu);
    std::vector<Fork>& set = fork_set[dev];
    Fork* f = nullptr;
    for (Fork& x : set) if (x.st == st) { f = &x; break; }
    if (!f) {
        if ((int)set.size() >= MAXFORKS) return nullptr;
        if (set.capacity() < (size_t)MAXFORKS) set.reserve(MAXFORKS);       // entries never move
        Fork n{st, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
        if (hipStreamCreateWithFlags(&n.side, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&n.fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&n.join, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;                                               // (what was made is kept: a few handles)
        }
        set.push_back(n);
        f = &set.back();
    }
    if (two && !f->side2) {
        hipStream_t s2 = nullptr;
        hipEvent_t lanes = nullptr, join2 = nullptr;
        if (hipStreamCreateWithFlags(&s2, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&lanes, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&join2, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        f->lanes = lanes; f->join2 = join2; f->side2 = s2;                // (side2 last: it marks the three made)
    }
    return f;
}

template <int Q>
hipError_t launch(const pv_dev_cohort& D, const int64_t* wa, const int64_t* ws, uint32_t W, uint32_t bpw, uint64_t nslots, const uint8_t* rc,
                  int tokens, int apply_case, void* out, const int64_t* ids, int32_t* status, uint8_t* slotbuf, HeavyList HL,
                  const SampleIn& X, hipEvent_t ev_mid, hipEvent_t ev_end, hipStream_t st, bool may_fork) {
    bool dec = true;                                    // windows_kernel with the wave decoder
    uint32_t xshift = ~0u;
    const Fork* fs = nullptr;                           // spill_kernel on a side stream, joined after windows_kernel
    const Fork* fh = nullptr;                           // heavy_kernel on a side stream, joined after windows_kernel
    if (slotbuf && (nslots <= small_slots<Q>() || !HL.cap)) {
        // one kernel: the heavy role's waves (one per slot; none without a heavy list), then the light waves
        auto fk = (nslots == bpw && nslots <= WAVE) ? front_kernel<Q, true> : front_kernel<Q, false>;   // one window: its table in LDS
        hipLaunchKernelGGL(fk, dim3(HL.nworkers + HL.nlight), dim3(WAVE), 0, st, D, wa, ws, W, bpw, nslots, slotbuf, X, HL);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        xshift = HL.nworkers & 7u;
    } else if (slotbuf) {
        // the slots' headers and the heavy list, then the heavy waves (Q <= 4096: one per heavy area) and the light
        // waves (one lane per slot), then the slots left to spill_kernel (at Q = 16384, which has no heavy areas, every
        // long block); windows_kernel then only replays
        dec = false;
        xshift = 0;
        // (at Q = 16384 a timed call stays on st: its side streams would join after the windows kernel's end event)
        // (timing with ev_mid brackets the windows kernel alone, so the call then keeps to one order; with ev_end only,
        // the end event follows the whole call and its joins)
        const Fork* f = (PV_FORK && may_fork && (Cfg<Q>::REGOPS || !ev_mid)) ? fork_of(st, !Cfg<Q>::REGOPS) : nullptr;
        // the fork and join events are bound to the kernels they follow (the launch's stop event) rather than recorded
        // after them: a recorded event is a packet of its own in the queue, which the queue's next kernel waits behind
        if (f) hipExtLaunchKernelGGL((slot_kernel<Q>), dim3(HL.nlight), dim3(WAVE), 0, st, nullptr, f->fork, 0u, D, wa, ws, W, bpw, nslots, slotbuf, X, HL);
        else hipLaunchKernelGGL((slot_kernel<Q>), dim3(HL.nlight), dim3(WAVE), 0, st, D, wa, ws, W, bpw, nslots, slotbuf, X, HL);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess && f) e = hipStreamWaitEvent(f->side, f->fork, 0);
        if (e != hipSuccess) return e;
        const uint32_t sw = spill_waves(nslots, HL.nworkers);
        if constexpr (Cfg<Q>::REGOPS) {
            if (f && !ev_mid) {
                // forked and untimed: each heavy wave replays its slot as soon as it has decoded it, beside the light
                // lanes and the replay of the light slots (which leaves them: skip_heavy) and the whole-slot pass on
                // the call's stream; the slots are disjoint, and so are the row bytes they write
                auto hk = (D.form & PV_FORM_PACKED_REF) ? heavy_replay_fused_kernel<Q, false> : heavy_replay_fused_kernel<Q, PV_LITE != 0>;
                hipExtLaunchKernelGGL(hk, dim3(HL.nworkers), dim3(WAVE), 0, f->side, nullptr, f->join, 0u, D, wa, ws, W, bpw, X, HL, rc, tokens,
                                      apply_case, out, ids, (int*)status, (const uint8_t*)slotbuf);
            } else if (f) {
                hipExtLaunchKernelGGL((heavy_kernel<Q>), dim3(HL.nworkers), dim3(WAVE), 0, f->side, nullptr, f->join, 0u, D, wa, ws, W, bpw, X, HL);
            } else {
                hipLaunchKernelGGL((heavy_kernel<Q>), dim3(HL.nworkers), dim3(WAVE), 0, st, D, wa, ws, W, bpw, X, HL);
            }
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL((light_decode_kernel<Q>), dim3(HL.nlight), dim3(WAVE), 0, st, D, wa, ws, W, bpw, nslots, slotbuf, X, HL);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            if (f && !ev_mid) {
                fh = f;       // the whole-slot pass and the join follow the replay (below)
            } else {
                if (f) e = hipStreamWaitEvent(st, f->join, 0);
                if (e != hipSuccess) return e;
                hipLaunchKernelGGL((spill_kernel<Q>), dim3(sw), dim3(WAVE), 0, st, D, wa, ws, W, bpw, X, HL, rc, tokens, apply_case, out, ids,
                                   (int*)status, (uint32_t)SPILL_ALL);
                e = hipGetLastError();
                if (e != hipSuccess) return e;
            }
        } else {
            // no heavy areas: a side stream does the list's long blocks whole from the start, beside the light lanes;
            // a second one the lanes' spilled slots once the lanes are done; both beside the replay (which leaves all
            // those slots to them) and joined after it
            if (f) hipExtLaunchKernelGGL((spill_kernel<Q>), dim3(sw), dim3(WAVE), 0, f->side, nullptr, f->join, 0u, D, wa, ws, W, bpw, X, HL, rc,
                                         tokens, apply_case, out, ids, (int*)status, (uint32_t)SPILL_LIST);
            else hipLaunchKernelGGL((spill_kernel<Q>), dim3(sw), dim3(WAVE), 0, st, D, wa, ws, W, bpw, X, HL, rc, tokens, apply_case, out, ids,
                                    (int*)status, (uint32_t)SPILL_LIST);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            if (f) hipExtLaunchKernelGGL((light_decode_kernel<Q>), dim3(HL.nlight), dim3(WAVE), 0, st, nullptr, f->lanes, 0u, D, wa, ws, W, bpw,
                                         nslots, slotbuf, X, HL);
            else hipLaunchKernelGGL((light_decode_kernel<Q>), dim3(HL.nlight), dim3(WAVE), 0, st, D, wa, ws, W, bpw, nslots, slotbuf, X, HL);
            e = hipGetLastError();
            if (e == hipSuccess && f) e = hipStreamWaitEvent(f->side2, f->lanes, 0);
            if (e != hipSuccess) return e;
            if (f) hipExtLaunchKernelGGL((spill_kernel<Q>), dim3(sw), dim3(WAVE), 0, f->side2, nullptr, f->join2, 0u, D, wa, ws, W, bpw, X, HL, rc,
                                         tokens, apply_case, out, ids, (int*)status, (uint32_t)SPILL_LANES);
            else hipLaunchKernelGGL((spill_kernel<Q>), dim3(sw), dim3(WAVE), 0, st, D, wa, ws, W, bpw, X, HL, rc, tokens, apply_case, out, ids,
                                    (int*)status, (uint32_t)SPILL_LANES);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            fs = f;
        }
    }
    // on the heavy-list path every slot arrives decoded (by a light lane or into a heavy area) or done whole: the
    // windows kernel then has no decoder
    // the replay-only kernel reads the reference from HBM where it is held as bytes (its LDS holds only the block)
    // (at Q = 16384, windows of at most WIN_W bases: the replay with the window buffer)
    const bool winbuf = !dec && !(D.form & PV_FORM_PACKED_REF) && !Cfg<Q>::REGOPS && PV_LITE && W <= WIN_W;
    auto kern = dec ? windows_kernel<Q, true> : (D.form & PV_FORM_PACKED_REF) ? windows_kernel<Q, false>
              : winbuf ? windows_kernel<Q, false, PV_LITE != 0, !Cfg<Q>::REGOPS>
              : windows_kernel<Q, false, PV_LITE != 0>;
    using WinLds = LdsLite<Q, true>;
    const size_t dyn = winbuf ? offsetof(WinLds, blk) + win_bytes(W) + 4 * lower_words(W) : 0;     // the window buffer's LDS
    if (ev_mid && ev_end) {
        // timing: the runtime sets the two events to the windows kernel's own start and end
        hipExtLaunchKernelGGL(kern, dim3((uint32_t)nslots), dim3(WAVE), dyn, st, ev_mid, ev_end, 0u, D, wa, ws, W, bpw, rc,
                              tokens, apply_case, out, ids, (int*)status, (const uint8_t*)slotbuf, (const uint64_t*)HL.done, (const uint8_t*)HL.area, xshift, HL.epoch,
                              fh ? 1u : 0u);
    } else {
        if (ev_mid) { const hipError_t e = hipEventRecord(ev_mid, st); if (e != hipSuccess) return e; }
        hipLaunchKernelGGL(kern, dim3((uint32_t)nslots), dim3(WAVE), dyn, st, D, wa, ws, W, bpw, rc, tokens, apply_case, out,
                           ids, (int*)status, (const uint8_t*)slotbuf, (const uint64_t*)HL.done, (const uint8_t*)HL.area, xshift, HL.epoch,
                           fh ? 1u : 0u);
    }
    if constexpr (Cfg<Q>::REGOPS) {
        if (fh) {
            hipLaunchKernelGGL((spill_kernel<Q>), dim3(spill_waves(nslots, HL.nworkers)), dim3(WAVE), 0, st, D, wa, ws, W, bpw, X, HL, rc,
                               tokens, apply_case, out, ids, (int*)status, (uint32_t)SPILL_ALL);
            hipError_t e = hipGetLastError();
            if (e == hipSuccess) e = hipStreamWaitEvent(st, fh->join, 0);      // the heavy waves and their slots' replay
            if (e != hipSuccess) return e;
        }
    }
    if (fs) {
        hipError_t e = hipStreamWaitEvent(st, fs->join, 0);
        if (e == hipSuccess) e = hipStreamWaitEvent(st, fs->join2, 0);
        if (e != hipSuccess) return e;
    }
    if (ev_end && !ev_mid) { const hipError_t e = hipEventRecord(ev_end, st); if (e != hipSuccess) return e; }   // the whole call
    return hipGetLastError();
}

// A number per launch that no earlier launch of this process used (never 0, which a zeroed buffer holds).
std::atomic<uint32_t> launch_epoch{0};
uint32_t next_epoch() { uint32_t e; do e = ++launch_epoch; while (e == 0); return e; }

}  // namespace

// Slot records of the light-block path for n windows of W bases (0: the block size does not use it)
static uint64_t light_scratch_bytes(uint32_t Q, int64_t n, int64_t W) {
    if (!(Q == 1024 || Q == 2048 || Q == 4096 || Q == 16384) || n <= 0 || W <= 0) return 0;
    return (uint64_t)n * (((uint64_t)W + Q - 1) / Q + 1) * SLOT_BYTES;
}
// Heavy areas of a call of nslots slots: one per slot up to SMALL_SLOTS (front_kernel's area `slot`); beyond, one per 64
// slots, at least 256 (heavy slots are a few per thousand in cohorts of long haplotypes; those past the count go to
// spill_kernel, which does them whole)
static uint64_t heavy_areas(uint64_t nslots) {
    if (nslots <= SMALL_SLOTS) return nslots;    // front_kernel: area `slot`
    const uint64_t a = nslots / 64 > 256 ? nslots / 64 : 256;
    return a < nslots ? a : nslots;
}
static uint64_t heavy_area_size(uint32_t Q) {
    return Q == 1024 ? Heavy<1024>::BYTES : Q == 2048 ? Heavy<2048>::BYTES : Q == 4096 ? Heavy<4096>::BYTES : 0;
}
// Bytes of the heavy list after the slot records (256-byte aligned): control words, per slot an entry and a done word,
// then the heavy areas (256-byte aligned)
static uint64_t heavy_area_bytes(uint32_t Q, int64_t n, int64_t W) {
    const uint64_t light = light_scratch_bytes(Q, n, W);
    if (!light) return 0;
    const uint64_t nslots = light / SLOT_BYTES;           // (Q = 16384: the list and done words, no areas)
    return ((light + 255) & ~255ull) - light + 256 + ((16 * nslots + 255) & ~255ull) + heavy_areas(nslots) * heavy_area_size(Q);
}
static uint64_t work_bytes_for(uint32_t Q, int64_t n, int64_t W) { return light_scratch_bytes(Q, n, W) + heavy_area_bytes(Q, n, W); }

// Whether a call may launch on stream st: not while the stream is being captured into a graph. A call that uses the
// work buffer marks its list, counter and done words with a number the host draws per launch (next_epoch), which a
// replayed graph would repeat; the words of an earlier replay would then read as this one's. So such calls refuse
// capture (PV_EARG), and so does sample on a caller stream under capture (its ring wait is host state per call).
static int32_t refuse_capture(hipStream_t st, char* err, size_t errcap) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) { (void)hipGetLastError(); seterr(err, errcap, "stream capture status unavailable (a graph capture in progress?)"); return PV_EARG; }
    if (cs != hipStreamCaptureStatusNone) {
        seterr(err, errcap, "stream is being captured into a graph: a decode call that uses the work buffer cannot be replayed from a graph");
        return PV_EARG;
    }
    return PV_OK;
}

// X: the sampler's inputs when light_decode_kernel computes the windows' coordinates (the light path must then be
// taken: the caller checked light_scratch_bytes), else nullptr
static int32_t windows_any(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W, const uint8_t* rc,
                           int32_t tokens, int32_t apply_case, void* out, const int64_t* ids, int32_t* status, void* work,
                           uint64_t work_bytes, const SampleIn* X, void* stream, char* err, size_t errcap, void* ev_mid = nullptr,
                           void* ev_end = nullptr, bool may_fork = true) {
    if (!D || (!asm_idx && n) || (!start && n) || !status || (!out && n && W)) { seterr(err, errcap, "null argument"); return PV_EARG; }
    const uint32_t Q = D->Q;
    if (!(Q == 1024 || Q == 2048 || Q == 4096 || Q == 16384)) { seterr(err, errcap, "block size"); return PV_EARG; }
    if (W < 0 || W >= (1ll << 31)) { seterr(err, errcap, "W"); return PV_EARG; }
    if (n < 0) { seterr(err, errcap, "n"); return PV_EARG; }
    if (n == 0 || W == 0) {                 // nothing to launch: the timing events still mark the (empty) call
        hipError_t e = hipSuccess;
        if (ev_mid) e = hipEventRecord((hipEvent_t)ev_mid, (hipStream_t)stream);
        if (e == hipSuccess && ev_end) e = hipEventRecord((hipEvent_t)ev_end, (hipStream_t)stream);
        if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
        return PV_OK;
    }
    const uint64_t bpw = ((uint64_t)W + Q - 1) / Q + 1;
    if ((uint64_t)n * bpw >= (1ull << 31)) { seterr(err, errcap, "too many blocks in one call (windows x blocks per window >= 2^31)"); return PV_EARG; }
    const uint64_t nslots = (uint64_t)n * bpw;
    const uint64_t need = light_scratch_bytes(Q, n, W);
    if (work && ((uintptr_t)work & 15)) { seterr(err, errcap, "work buffer not 16-byte aligned"); return PV_EARG; }
    uint8_t* slotbuf = (work && need && work_bytes >= need) ? (uint8_t*)work : nullptr;
    // a call of one or two slots at Q = 16384 (a fetch) is one block's serial decode: the wave decoder does it and the
    // replay in one kernel, where the light lanes would add a launch and a slot record's round trip
    if (Q == 16384 && nslots <= 2 && !X) slotbuf = nullptr;
    if (X && !slotbuf) { seterr(err, errcap, "sampler coordinates need the light-block slot records"); return PV_EARG; }
    if (slotbuf) {
        const int32_t cap = refuse_capture((hipStream_t)stream, err, errcap);
        if (cap) return cap;
    }
    // with room for the heavy list too, long blocks are done by heavy waves beside the light lanes' decode
    HeavyList HL{};
    HL.nlight = (uint32_t)((nslots + WAVE - 1) / WAVE);
    HL.epoch = next_epoch();
    if (slotbuf && work_bytes >= work_bytes_for(Q, n, W)) {
        uint8_t* h = (uint8_t*)work + ((need + 255) & ~255ull);
        HL.cap = (uint32_t)nslots;
        HL.ctl = (HeavyCtl*)h;
        HL.list = (uint64_t*)(h + 256);
        HL.done = HL.list + nslots;
        HL.area = h + 256 + ((16 * nslots + 255) & ~255ull);
        HL.acap = heavy_area_size(Q) ? (uint32_t)heavy_areas(nslots) : 0u;   // none at Q = 16384
        HL.nworkers = HL.acap;           // heavy_kernel: one wave per area (front_kernel's heavy role: one per slot)
    }
    SampleIn none{};
    const SampleIn& XX = X ? *X : none;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    switch (Q) {
        case 1024: e = launch<1024>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, ids, status, slotbuf, HL, XX, (hipEvent_t)ev_mid, (hipEvent_t)ev_end, st, may_fork); break;
        case 2048: e = launch<2048>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, ids, status, slotbuf, HL, XX, (hipEvent_t)ev_mid, (hipEvent_t)ev_end, st, may_fork); break;
        case 4096: e = launch<4096>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, ids, status, slotbuf, HL, XX, (hipEvent_t)ev_mid, (hipEvent_t)ev_end, st, may_fork); break;
        default: e = launch<16384>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, ids, status, slotbuf, HL, XX, (hipEvent_t)ev_mid, (hipEvent_t)ev_end, st, may_fork); break;
    }
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    return PV_OK;
}

// The kernels' four-bytes-at-a-time transforms against the per-byte definitions, on the host: every byte value in
// every byte lane beside 256 neighbour patterns, for comp4, comp_case4 and token4, and all 16 flag sets for case4.
// Returns the number of mismatches.
extern "C" int32_t pv_selftest_bytes(void) {
    int32_t bad = 0;
    for (uint32_t b = 0; b < 256; b++)
        for (uint32_t k = 0; k < 4; k++)
            for (uint32_t o = 0; o < 256; o++) {
                const uint32_t other = o * 0x01010101u ^ 0x5A3C0F96u;           // the other three bytes vary too
                const uint32_t w = (other & ~(0xFFu << (8 * k))) | (b << (8 * k));
                const uint32_t c = comp4(w), cc = comp_case4(w), t = token4(w);
                for (uint32_t i = 0; i < 4; i++) {
                    const uint8_t x = (uint8_t)(w >> (8 * i));
                    bad += (uint8_t)(c >> (8 * i)) != pvc::comp(x);
                    bad += (uint8_t)(cc >> (8 * i)) != pvc::comp_case(x);
                    bad += (uint8_t)(t >> (8 * i)) != pvc::token(x);
                }
            }
    for (uint32_t f = 0; f < 16; f++)
        for (uint32_t i = 0; i < 4; i++) bad += ((case4(f) >> (8 * i)) & 0xFFu) != (((f >> i) & 1u) ? 0x20u : 0u);
    return bad;
}

extern "C" uint64_t pv_windows_work_bytes(const pv_dev_cohort* D, int64_t n, int64_t W) {
    return D ? work_bytes_for(D->Q, n, W) : 0;
}

extern "C" int32_t pv_windows_hip(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W, const uint8_t* rc,
                                  int32_t tokens, int32_t apply_case, uint8_t* out, int32_t* status, void* work, uint64_t work_bytes,
                                  void* stream, char* err, size_t errcap) {
    return windows_any(D, asm_idx, start, n, W, rc, tokens, apply_case, out, nullptr, status, work, work_bytes, nullptr, stream, err, errcap);
}

extern "C" int32_t pv_windows_ids_hip(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W, const uint8_t* rc,
                                      const int64_t* ids, int64_t* out, int32_t* status, void* work, uint64_t work_bytes, void* stream,
                                      char* err, size_t errcap) {
    if (!ids) { seterr(err, errcap, "null argument"); return PV_EARG; }
    return windows_any(D, asm_idx, start, n, W, rc, 1, 0, out, ids, status, work, work_bytes, nullptr, stream, err, errcap);
}

namespace {
// One window's coordinates from kernel arguments into the call's coordinate record (assembly, start, strand byte) and
// its status word zeroed: what two host-to-device copies and a fill did, in one launch that the host does not wait for
__global__ void __launch_bounds__(WAVE) fetch_coord_kernel(int64_t* rec, int64_t a, int64_t s, uint32_t rc) {
    if (threadIdx.x == 0) {
        rec[0] = a; rec[1] = s;
        rec[2] = (int64_t)(rc ? 1 : 0);                 // the strand byte (the record's byte 16) and zeros after it
        rec[3] = 0;                                     // the status word (byte 24) and padding
    }
}
}  // namespace

extern "C" int32_t pv_fetch_hip(const pv_dev_cohort* D, int64_t assembly, int64_t start, int64_t W, int32_t rc, int32_t tokens,
                                uint8_t* out, void* rec, void* work, uint64_t work_bytes, void* stream, char* err, size_t errcap) {
    if (!D || !rec || (!out && W)) { seterr(err, errcap, "null argument"); return PV_EARG; }
    if ((uintptr_t)rec & 15) { seterr(err, errcap, "coordinate record not 16-byte aligned"); return PV_EARG; }
    if (W < 0 || W >= (1ll << 31)) { seterr(err, errcap, "W"); return PV_EARG; }
    int64_t* R = (int64_t*)rec;
    const uint32_t Q = D->Q;
    if (W > 0 && Q != 16384 && work && light_scratch_bytes(Q, 1, W) && work_bytes >= light_scratch_bytes(Q, 1, W)) {
        // the decode kernel takes the coordinates as arguments and writes the record itself: one launch fewer
        SampleIn X{};
        X.fixed = 1; X.fa = assembly; X.fs = start; X.rcmode = rc ? 1 : 0;
        X.wasm = R; X.wstart = R + 1; X.wrc = (uint8_t*)(R + 2); X.status = (int*)(R + 3);
        return windows_any(D, R, R + 1, 1, W, rc ? (const uint8_t*)(R + 2) : nullptr, tokens, 1, out, nullptr, (int32_t*)(R + 3), work,
                           work_bytes, &X, stream, err, errcap);
    }
    hipLaunchKernelGGL(fetch_coord_kernel, dim3(1), dim3(WAVE), 0, (hipStream_t)stream, R, assembly, start, (uint32_t)(rc != 0));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    return windows_any(D, R, R + 1, 1, W, rc ? (const uint8_t*)(R + 2) : nullptr, tokens, 1, out, nullptr, (int32_t*)(R + 3), work,
                       work_bytes, nullptr, stream, err, errcap);
}

// The work buffer of pv_windows_hip_noalloc: one array per GPU the library runs on, held until the process ends. Host
// code never passes the array's name to a kernel (on the host it stands for a host-side shadow, not device memory):
// each device's address comes from hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) uint8_t scratch[PV_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex scratch_mu;
void* scratch_dev[64];                        // the array's address on each device, nullptr until first looked up
}  // namespace

extern "C" int32_t pv_launch_prepare(const pv_dev_cohort* D, int64_t n, int64_t W, void* stream, char* err, size_t errcap) {
    if (!D) { seterr(err, errcap, "null argument"); return PV_EARG; }
    const uint32_t Q = D->Q;
    if (n <= 0 || W <= 0 || W >= (1ll << 31) || !(Q == 1024 || Q == 2048 || Q == 4096 || Q == 16384)) return PV_OK;
    const uint64_t nslots = (uint64_t)n * (((uint64_t)W + Q - 1) / Q + 1);
    if (PV_FORK && nslots > (Q == 16384 ? SMALL_SLOTS_Q16 : SMALL_SLOTS) && nslots < (1ull << 31))
        (void)fork_of((hipStream_t)stream, Q == 16384);                  // else: one stream
    return PV_OK;
}

extern "C" int32_t pv_windows_hip_noalloc(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W,
                                          const uint8_t* rc, int32_t tokens, int32_t apply_case, uint8_t* out, int32_t* status,
                                          void* stream, char* err, size_t errcap) {
    if (!D) { seterr(err, errcap, "null argument"); return PV_EARG; }
    const uint32_t Q = D->Q;
    uint64_t need = (W > 0 && W < (1ll << 31) && n > 0 && (uint64_t)n < (1ull << 31)) ? light_scratch_bytes(Q, n, W) : 0;
    if (need > PV_NOALLOC_SCRATCH_BYTES && Q == 16384) need = 0;   // the wave decoder alone, which needs no scratch
    if (need > PV_NOALLOC_SCRATCH_BYTES) {
        char m[256];
        snprintf(m, sizeof m, "pv_windows_hip_noalloc: %llu windows of %lld bases need %llu bytes of scratch, over the %u this entry "
                 "point holds (use pv_windows_hip with a work buffer)", (unsigned long long)n, (long long)W, (unsigned long long)need,
                 (unsigned)PV_NOALLOC_SCRATCH_BYTES);
        seterr(err, errcap, m);
        return PV_EARG;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= 64)) e = hipErrorInvalidDevice;
    void* ptr = nullptr;
    if (e == hipSuccess) {
        std::lock_guard<std::mutex> g(scratch_mu);
        if (!scratch_dev[dev]) {
            e = hipGetSymbolAddress(&scratch_dev[dev], HIP_SYMBOL(scratch));
            if (e != hipSuccess) scratch_dev[dev] = nullptr;
        }
        ptr = scratch_dev[dev];
    }
    if (e != hipSuccess || !ptr) { seterr(err, errcap, e != hipSuccess ? hipGetErrorString(e) : "scratch address"); return PV_EHIP; }
    // the light-block slots, and the heavy areas after them where they fit too; no part must start at zero (every
    // slot's header is written before it is read, and a heavy area is read only for a slot whose header says it was
    // written)
    const uint64_t all = work_bytes_for(Q, n, W);
    return windows_any(D, asm_idx, start, n, W, rc, tokens, apply_case, out, nullptr, status, need ? ptr : nullptr,
                       !need ? 0 : all <= PV_NOALLOC_SCRATCH_BYTES ? all : need, nullptr, stream, err, errcap, nullptr, nullptr,
                       false);             // no stream of the library's own: the kernels one after another
}

static int32_t sample_args_check(const int64_t* cum, int64_t ncontigs, const int64_t* ctg_asm, const int64_t* ctg_local,
                                 const int64_t* ctg_boff, const int64_t* draws, const float* rnd, int32_t rcmode, int64_t n,
                                 const int64_t* wasm, const int64_t* wstart, const uint8_t* wrc, const int32_t* status, char* err,
                                 size_t errcap) {
    if (!status || (n && (!cum || !ctg_asm || !ctg_local || !ctg_boff || !draws || !wasm || !wstart)) || (rcmode && n && !wrc) ||
        (rcmode == 2 && n && !rnd)) {
        seterr(err, errcap, "null argument"); return PV_EARG;
    }
    if (rcmode < 0 || rcmode > 2) { seterr(err, errcap, "rcmode"); return PV_EARG; }
    if (ncontigs <= 0) { seterr(err, errcap, "no contigs"); return PV_EARG; }
    if (n < 0 || n >= (1ll << 40)) { seterr(err, errcap, "n"); return PV_EARG; }
    return PV_OK;
}

extern "C" int32_t pv_sample_coords_hip(const int64_t* cum, int64_t ncontigs, const int64_t* ctg_asm, const int64_t* ctg_local,
                                        const int64_t* ctg_boff, const int64_t* draws, const float* rnd, double p, int32_t rcmode, int64_t n,
                                        int64_t* wasm, int64_t* wstart, uint8_t* wrc, int64_t* coords, int32_t* status, void* stream,
                                        char* err, size_t errcap) {
    const int32_t bad = sample_args_check(cum, ncontigs, ctg_asm, ctg_local, ctg_boff, draws, rnd, rcmode, n, wasm, wstart, wrc, status, err, errcap);
    if (bad) return bad;
    const int64_t per = 256 / WAVE;
    const int64_t blocks = n > 0 ? (n + per - 1) / per : 1;
    if (blocks >= (1ll << 31)) { seterr(err, errcap, "n"); return PV_EARG; }
    hipLaunchKernelGGL(sample_coords_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, cum, ncontigs, draws, rnd, (float)p,
                       rcmode, ctg_asm, ctg_local, ctg_boff, n, wasm, wstart, wrc, coords, (int*)status);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    return PV_OK;
}

namespace {
// How a caller's stream is made to wait for work the library enqueued on another stream (the lane), and how far the
// host may run ahead of the caller's stream.
// PV_WAIT_COUNTER: a 64-bit counter per lane in signal memory, which the lane advances after each call's kernels
// (hipStreamWriteValue64); on the caller's stream one small kernel (caller_wait_kernel) polls it until the call's mark,
// then stores the caller's own mark. One dispatch per call on the caller's queue: the caller's queue passes calls at
// about twice the rate it does with the runtime's wait-value and write-value operations (each a dispatch of its own),
// and that rate bounds how many calls the ring keeps in flight. The poll would wait for a lane kernel that cannot start
// where dispatches are serialised (counter collection), so the counter wait is not used there. A lane executes its
// calls in order, so its counter only grows.
// PV_WAIT_EVENT: events, one per call in turn from a small ring per lane, recorded on the lane and waited for by the
// caller (hipStreamWaitEvent takes the event's state at the time of the call); ~20 us of host time per call.
// Backpressure: after its wait, the caller's stream marks its progress (its own counter, or an event of a ring of
// CALLER_DEPTH), and a call first waits on the host until the caller's stream has passed all but CALLER_DEPTH - 1 of
// the earlier calls (at most LANE_SPIN_S seconds). The caller's stream passes calls in order, and what it frees after
// a call becomes reusable once it has passed that call; so a host thread that enqueues faster than the GPU decodes
// holds at most CALLER_DEPTH calls and their rows in flight, whatever the ring size.
// One mutex per device keeps a call's launches, its counter write or event and its waits together. Falls back to
// events where the device lacks stream wait-value support or signal memory cannot be had. Signal memory and events
// are kept for the life of the process.
constexpr int MAXLANES = 256, LANE_EVENTS = 4, CALLER_DEPTH = 32;
constexpr double LANE_SPIN_S = 60.0;
// The caller's wait for a lane's mark (one lane of one wave): poll the lane's counter (system scope: signal memory
// that another queue's packet writes) until it reaches `target`, then store the caller's mark `mark`. Bounded at
// LANE_SPIN_S of the GPU's 100 MHz clock: past it the wave stores the mark anyway and sets status bit 4 in the call's
// status word, so that the call reports the wait instead of returning rows that may not be complete.
constexpr uint64_t WAIT_TICKS = (uint64_t)(LANE_SPIN_S * 100e6);
__global__ void __launch_bounds__(WAVE) caller_wait_kernel(const uint64_t* lane, uint64_t target, uint64_t* mark, uint64_t m, int* status) {
    if (threadIdx.x != 0) return;
    const uint64_t t0 = wall_clock64();
    while (__hip_atomic_load(lane, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) < target) {
        if (wall_clock64() - t0 > WAIT_TICKS) { atomicOr(status, PV_ST_WAIT); break; }
        __builtin_amdgcn_s_sleep(2);
    }
    __hip_atomic_store(mark, m, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}
struct Sig {                                              // a lane's or a caller's progress marks
    hipStream_t s;
    uint64_t* p;                                          // counter in signal memory, or nullptr: events
    uint64_t n;                                           // marks made
    hipEvent_t ev[CALLER_DEPTH];                          // the event of mark m is ev[m % nev]
    int nev;
};
struct DevSync {
    std::mutex mu;
    int mode = -1;                                        // -1 not probed, 0 events, 1 counters
    std::vector<Sig> lanes, callers;                      // reserved for MAXLANES each: entries never move
};
std::mutex sync_mu;
DevSync* dev_sync[64];
DevSync* sync_of(int dev) {
    std::lock_guard<std::mutex> g(sync_mu);
    if (!dev_sync[dev]) {
        dev_sync[dev] = new DevSync();
        dev_sync[dev]->lanes.reserve(MAXLANES); dev_sync[dev]->callers.reserve(MAXLANES);
    }
    return dev_sync[dev];
}
// A tool that serialises kernel dispatches (rocprofv3 counter collection or thread trace, which set these variables for
// the process they profile): a caller wait carried out as a polling kernel would then wait for a lane kernel that
// cannot start until the poll ends, so the counter wait falls back to events there.
bool serialised_dispatch() {
    static const bool on = [] {
        for (const char* v : {"ROCPROF_COUNTER_COLLECTION", "ROCPROF_COUNTERS", "ROCPROF_COUNTER_GROUPS", "ROCPROF_ADVANCED_THREAD_TRACE"}) {
            const char* s = getenv(v);
            if (s && *s && strcmp(s, "0") != 0 && strcasecmp(s, "false") != 0) return true;
        }
        return false;
    }();
    return on;
}
// The marks of stream st in `set` (lanes or callers), created on first use with nev events (with S.mu held); with
// `counter` (and stream wait-value support) also a counter, zeroed before any wait can read it - signal memory does not
// start at 0, and a zeroing write only enqueued could land after a first wait had read the old value. nullptr on a HIP
// error (err set).
Sig* sig_state(DevSync& S, std::vector<Sig>& set, int dev, hipStream_t st, int nev, bool counter, hipError_t& err) {
    err = hipSuccess;
    Sig* L = nullptr;
    for (auto& x : set) if (x.s == st) L = &x;
    if (L && (L->p || !counter || S.mode == 0)) return L;
    if (counter && S.mode < 0) {
        int v = 0;
        S.mode = (hipDeviceGetAttribute(&v, hipDeviceAttributeCanUseStreamWaitValue, dev) == hipSuccess && v) ? 1 : 0;
    }
    if (!L) {
        if ((int)set.size() >= MAXLANES) { err = hipErrorOutOfMemory; return nullptr; }
        Sig z{};
        z.s = st; z.nev = nev;
        for (int i = 0; i < nev && err == hipSuccess; i++) err = hipEventCreateWithFlags(&z.ev[i], hipEventDisableTiming);
        if (err != hipSuccess) return nullptr;
        set.push_back(z);
        L = &set.back();
    }
    if (counter && S.mode == 1 && !L->p) {
        void* p = nullptr;
        if (hipExtMallocWithFlags(&p, 8, hipMallocSignalMemory) != hipSuccess || !p) { (void)hipGetLastError(); S.mode = 0; return L; }
        // the counter takes over from the events once what they covered is done (counter 0: nothing in flight)
        if (hipStreamSynchronize(st) != hipSuccess || hipStreamWriteValue64(st, p, 0, 0) != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
            (void)hipGetLastError(); S.mode = 0; return L;
        }
        L->p = (uint64_t*)p; L->n = 0;
    }
    return L;
}
// Backpressure before mark C.n + 1 of a caller (with S.mu held): wait until its mark C.n + 1 - C.nev is reached.
hipError_t sig_room(Sig& C) {
    if (C.n + 1 <= (uint64_t)C.nev) return hipSuccess;
    const uint64_t need = C.n + 1 - (uint64_t)C.nev;
    if (!C.p) return hipEventSynchronize(C.ev[(C.n + 1) % C.nev]);
    const volatile uint64_t* c = C.p;
    if (*c >= need) return hipSuccess;
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t k = 0; *c < need; k++) {
        if (k > 64) std::this_thread::yield();
        if ((k & 1023) == 0 && std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > LANE_SPIN_S)
            return hipErrorLaunchTimeOut;
    }
    return hipSuccess;
}
// Mark C.n + 1 on its stream, after everything enqueued there so far: the counter when there is one (so that it always
// equals the marks made), and the mark's event where there is no counter or `event` asks for it.
hipError_t sig_mark(Sig& C, bool event) {
    C.n++;
    hipError_t e = hipSuccess;
    if (C.p) e = hipStreamWriteValue64(C.s, C.p, C.n, 0);
    if (e == hipSuccess && (!C.p || event)) e = hipEventRecord(C.ev[C.n % C.nev], C.s);
    return e;
}
}  // namespace

extern "C" int32_t pv_dispatch_serialised(void) { return serialised_dispatch() ? 1 : 0; }

namespace {
// One lane waits until the GPU's real-time clock (100 MHz) has advanced `ticks`: a kernel of known length for
// pv_streams_concurrent, whose every wave ends.
__global__ void __launch_bounds__(WAVE) hold_kernel(uint64_t ticks) {
    if (threadIdx.x == 0) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(4);
    }
}
}  // namespace

extern "C" int32_t pv_streams_concurrent(void* a, void* b, int32_t* concurrent, char* err, size_t errcap) {
    if (!concurrent) { seterr(err, errcap, "null argument"); return PV_EARG; }
    *concurrent = 0;
    constexpr uint64_t TICKS = 10000;                   // 100 us
    const hipStream_t sa = (hipStream_t)a, sb = (hipStream_t)b;
    hipEvent_t e0 = nullptr, ea = nullptr, eb = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&ea);
    if (e == hipSuccess) e = hipEventCreate(&eb);
    if (e == hipSuccess) e = hipStreamSynchronize(sa);
    if (e == hipSuccess) e = hipStreamSynchronize(sb);
    if (e == hipSuccess) e = hipEventRecord(e0, sa);
    if (e == hipSuccess) e = hipStreamWaitEvent(sb, e0, 0);
    if (e == hipSuccess) { hipLaunchKernelGGL(hold_kernel, dim3(1), dim3(WAVE), 0, sa, TICKS); e = hipGetLastError(); }
    if (e == hipSuccess) { hipLaunchKernelGGL(hold_kernel, dim3(1), dim3(WAVE), 0, sb, TICKS); e = hipGetLastError(); }
    if (e == hipSuccess) e = hipEventRecord(ea, sa);
    if (e == hipSuccess) e = hipEventRecord(eb, sb);
    if (e == hipSuccess) e = hipEventSynchronize(ea);
    if (e == hipSuccess) e = hipEventSynchronize(eb);
    float ta = 0.f, tb = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ta, e0, ea);
    if (e == hipSuccess) e = hipEventElapsedTime(&tb, e0, eb);
    for (hipEvent_t x : {e0, ea, eb}) if (x) (void)hipEventDestroy(x);
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    // one after another: ~200 us from the release to the later end; at once: ~100 us and the launch gap
    *concurrent = std::max(ta, tb) < 1.5f * 1e-5f * (float)TICKS ? 1 : 0;
    return PV_OK;
}

extern "C" int32_t pv_sample_prepare(void* stream, void* caller, int32_t wait, char* err, size_t errcap) {
    if (wait != PV_WAIT_EVENT && wait != PV_WAIT_COUNTER) { seterr(err, errcap, "wait mode"); return PV_EARG; }
    if (stream == caller) return PV_OK;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= 64)) e = hipErrorInvalidDevice;
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    DevSync& S = *sync_of(dev);
    std::lock_guard<std::mutex> g(S.mu);
    const bool counter = wait == PV_WAIT_COUNTER && !serialised_dispatch();
    if (!sig_state(S, S.lanes, dev, (hipStream_t)stream, LANE_EVENTS, counter, e) ||
        !sig_state(S, S.callers, dev, (hipStream_t)caller, CALLER_DEPTH, counter, e)) {
        seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP;
    }
    return PV_OK;
}

extern "C" uint64_t pv_sample_work_bytes(const pv_dev_cohort* D, int64_t n, int64_t W) {
    return (((uint64_t)(n > 0 ? n : 0) * 17 + 255) & ~255ull) + (D ? work_bytes_for(D->Q, n, W) : 0);
}

extern "C" int32_t pv_sample_hip(const pv_dev_cohort* D, const int64_t* cum, int64_t ncontigs, const int64_t* ctg_asm, const int64_t* ctg_local,
                                 const int64_t* ctg_boff, const int64_t* draws, const float* rnd, double p, int32_t rcmode, int64_t n, int64_t W,
                                 int32_t tokens, int32_t apply_case, const int64_t* ids, void* work, uint64_t work_bytes, int64_t* coords,
                                 void* out, int32_t* status, void* stream, void* caller, int32_t wait, void* ev_start, void* ev_mid,
                                 void* ev_end, char* err, size_t errcap) {
    if (!D || (n && (!work || !out))) { seterr(err, errcap, "null argument"); return PV_EARG; }
    if (W <= 0 || W >= (1ll << 31)) { seterr(err, errcap, "W"); return PV_EARG; }
    if (wait != PV_WAIT_EVENT && wait != PV_WAIT_COUNTER) { seterr(err, errcap, "wait mode"); return PV_EARG; }
    if (((uintptr_t)work & 15) != 0) { seterr(err, errcap, "work buffer not 16-byte aligned"); return PV_EARG; }
    if (caller != stream) {
        const int32_t cap = refuse_capture((hipStream_t)caller, err, errcap);
        if (cap) return cap;
    }
    const uint64_t coord_bytes = ((uint64_t)n * 17 + 255) & ~255ull;   // window assembly, start, strand; then the scratch
    if (n && work_bytes < coord_bytes) { seterr(err, errcap, "work buffer smaller than pv_sample_work_bytes"); return PV_EARG; }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= 64)) e = hipErrorInvalidDevice;
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    DevSync& S = *sync_of(dev);
    std::lock_guard<std::mutex> g(S.mu);
    hipStream_t st = (hipStream_t)stream;
    Sig *L = nullptr, *C = nullptr;
    if (caller != stream) {                             // NULL is the null stream, which needs the wait too
        const bool counter = wait == PV_WAIT_COUNTER && !serialised_dispatch();
        L = sig_state(S, S.lanes, dev, st, LANE_EVENTS, counter, e);
        if (L) C = sig_state(S, S.callers, dev, (hipStream_t)caller, CALLER_DEPTH, counter, e);
        if (C) e = sig_room(*C);
        if (e != hipSuccess) {
            seterr(err, errcap, e == hipErrorLaunchTimeOut ? "sample: the caller's stream made no progress for 60 s" : hipGetErrorString(e));
            return PV_EHIP;
        }
    }
    int64_t* wa = (int64_t*)work;
    int64_t* ws = wa + n;
    uint8_t* wr = (uint8_t*)(ws + n);
    // with the light-block scratch, light_decode_kernel computes the coordinates itself; else a kernel of their own
    const uint64_t need = light_scratch_bytes(D->Q, n, W);
    const bool fused = n > 0 && need && work_bytes - coord_bytes >= need;
    int32_t code = PV_OK;
    SampleIn X{};
    if (fused) {
        code = sample_args_check(cum, ncontigs, ctg_asm, ctg_local, ctg_boff, draws, rnd, rcmode, n, wa, ws, rcmode ? wr : nullptr, status,
                                 err, errcap);
        X.cum = cum; X.nctg = ncontigs; X.draws = draws; X.rnd = rnd; X.p = (float)p; X.rcmode = rcmode; X.ctg_asm = ctg_asm;
        X.ctg_local = ctg_local; X.ctg_boff = ctg_boff; X.wasm = wa; X.wstart = ws; X.wrc = rcmode ? wr : nullptr; X.coords = coords;
        X.status = status;
    } else {
        code = pv_sample_coords_hip(cum, ncontigs, ctg_asm, ctg_local, ctg_boff, draws, rnd, p, rcmode, n, wa, ws, rcmode ? wr : nullptr,
                                    coords, status, stream, err, errcap);
    }
    if (code) return code;
    if (ev_start) e = hipEventRecord((hipEvent_t)ev_start, st);
    if (e == hipSuccess) {
        // a large call forks its heavy decode to a side stream only on the caller's own stream: on a ring stream the
        // calls already overlap, and a side stream per ring stream would pass the hardware queues HIP gives the
        // process, after which every stream's calls slow down (n = 1024 on the ring: 23.7 M windows/s, 13.8 M after
        // large calls had made the side streams, 8.0 M beside 15 more idle streams)
        code = windows_any(D, wa, ws, n, W, rcmode ? wr : nullptr, ids ? 1 : tokens, ids ? 0 : apply_case, out, ids, status,
                           (uint8_t*)work + coord_bytes, work_bytes - coord_bytes, fused ? &X : nullptr, stream, err, errcap, ev_mid,
                           ev_end, stream == caller);
        if (code) return code;
    }
    if (e == hipSuccess && L && C) {
        const bool counter = L->p && C->p && wait == PV_WAIT_COUNTER && !serialised_dispatch();
        // The lane's event too, with the counter: a stream whose last command is an event record is finished by a
        // device-wide synchronize through that event's signal, where after a kernel or a counter write the runtime
        // first sends a marker down the stream and waits for it (~16 us per stream with work, one after another).
        e = sig_mark(*L, true);
        if (e == hipSuccess && counter) {
            C->n++;                                     // the caller's mark, stored by its wait kernel
            hipLaunchKernelGGL(caller_wait_kernel, dim3(1), dim3(WAVE), 0, (hipStream_t)caller, (const uint64_t*)L->p, L->n, C->p, C->n,
                               (int*)status);
            e = hipGetLastError();
        } else if (e == hipSuccess) {
            e = hipStreamWaitEvent((hipStream_t)caller, L->ev[L->n % L->nev], 0);
            if (e == hipSuccess) e = sig_mark(*C, false);
        }
    }
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    return PV_OK;
}

extern "C" int32_t pv_sample_hip_call(const pv_sample_call* c) {
    if (!c) return PV_EARG;
    return pv_sample_hip(c->D, c->cum, c->ncontigs, c->ctg_asm, c->ctg_local, c->ctg_boff, c->draws, c->rnd, c->p, c->rcmode, c->n, c->W,
                         c->tokens, c->apply_case, c->ids, c->work, c->work_bytes, c->coords, c->out, c->status, c->stream, c->caller,
                         c->wait, c->ev_start, c->ev_mid, c->ev_end, c->err, (size_t)c->errcap);
}

namespace {
// ---- sample's rows from a pool of the library's own
//
// A call's rows are device memory that the caller's stream uses after the call. From torch's caching allocator they
// need record_stream, whose event the allocator records on the caller's stream when the tensor is freed: a second
// dispatch per call on the caller's queue, beside the wait. Rows from this pool are handed to torch as DLPack tensors
// instead; when torch frees one, its deleter notes the caller's next mark (the next call's wait kernel stores it, after
// every use the caller enqueued before the free), and the row is handed out again once the caller's counter has passed
// that mark. Pools live for the process (a deleter may run at any time, on any thread).
struct DLDeviceV { int32_t device_type, device_id; };
struct DLDataTypeV { uint8_t code, bits; uint16_t lanes; };
struct DLTensorV { void* data; DLDeviceV device; int32_t ndim; DLDataTypeV dtype; int64_t* shape; int64_t* strides; uint64_t byte_offset; };
struct DLManagedTensorV { DLTensorV dl_tensor; void* manager_ctx; void (*deleter)(DLManagedTensorV*); };
constexpr int32_t DL_ROCM = 10, DL_UINT = 1, DL_INT = 0;
struct RowPool;
struct Row {
    RowPool* pool;
    void* ptr;
    const Sig* caller;                 // the caller the row was last handed to (nullptr: never)
    uint64_t tag;                      // reusable once *caller->p >= tag
    int64_t shape[2];
    DLManagedTensorV mt;
};
struct RowPool {
    int dev;
    uint64_t bytes;
    std::mutex mu;
    std::vector<Row*> all;
    std::vector<Row*> free;            // oldest first
};
std::mutex pools_mu;
std::vector<RowPool*> pools;           // never freed
// rows of all pools of the process at most: a process that samples many shapes keeps a pool per row size, and a new
// size's reservation frees idle rows of the others to stay under this (calls past what it could reserve take torch's
// rows)
constexpr uint64_t ROWS_MAX_BYTES = 4ull << 30;
std::atomic<uint64_t> rows_bytes{0};
// Frees idle rows - never handed out, or handed back with the caller's counter past their mark - of the device's other
// pools, in the order the pools were made, until `need` more bytes fit under ROWS_MAX_BYTES. Set-up only (hipFree).
void rows_evict(const RowPool* keep, uint64_t need) {
    std::lock_guard<std::mutex> g(pools_mu);
    for (RowPool* p : pools) {
        if (rows_bytes.load() + need <= ROWS_MAX_BYTES) return;
        if (p == keep || p->dev != keep->dev) continue;
        std::lock_guard<std::mutex> g2(p->mu);
        for (size_t i = 0; i < p->free.size() && rows_bytes.load() + need > ROWS_MAX_BYTES;) {
            Row* x = p->free[i];
            const bool idle = !x->caller || __atomic_load_n((const uint64_t*)x->caller->p, __ATOMIC_ACQUIRE) >= x->tag;
            if (!idle || hipFree(x->ptr) != hipSuccess) { (void)hipGetLastError(); i++; continue; }
            rows_bytes -= p->bytes;
            p->free.erase(p->free.begin() + (std::ptrdiff_t)i);
            p->all.erase(std::find(p->all.begin(), p->all.end(), x));
            delete x;
        }
    }
}
void row_deleter(DLManagedTensorV* m) {
    Row* r = (Row*)m->manager_ctx;
    uint64_t tag = 0;
    if (r->caller) {
        DevSync& S = *sync_of(r->pool->dev);
        std::lock_guard<std::mutex> g(S.mu);
        tag = r->caller->n + 1;
    }
    std::lock_guard<std::mutex> g(r->pool->mu);
    r->tag = tag;
    r->pool->free.push_back(r);
}
}  // namespace

extern "C" int32_t pv_rows_reserve(uint64_t bytes, int32_t count, void** pool, char* err, size_t errcap) {
    if (!pool || !bytes || count < 0) { seterr(err, errcap, "argument"); return PV_EARG; }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    RowPool* P = nullptr;
    {
        std::lock_guard<std::mutex> g(pools_mu);
        for (RowPool* p : pools) if (p->dev == dev && p->bytes == bytes) P = p;
        if (!P) { P = new RowPool(); P->dev = dev; P->bytes = bytes; pools.push_back(P); }
    }
    uint64_t have = 0;
    { std::lock_guard<std::mutex> g(P->mu); have = P->all.size(); }
    if ((uint64_t)count > have) rows_evict(P, ((uint64_t)count - have) * bytes);
    std::lock_guard<std::mutex> g(P->mu);
    while ((int32_t)P->all.size() < count) {
        if (rows_bytes.fetch_add(bytes) + bytes > ROWS_MAX_BYTES) { rows_bytes -= bytes; break; }
        void* ptr = nullptr;
        e = hipMalloc(&ptr, bytes);
        if (e != hipSuccess) rows_bytes -= bytes;
        if (e != hipSuccess) { (void)hipGetLastError(); break; }          // fewer rows: calls past them use torch's
        Row* r = new Row{};
        r->pool = P; r->ptr = ptr;
        P->all.push_back(r);
        P->free.push_back(r);
    }
    *pool = P;
    return PV_OK;
}

extern "C" void* pv_rows_take(void* pool, void* caller, int64_t n, int64_t W, int32_t bits) {
    RowPool* P = (RowPool*)pool;
    if (!P || n <= 0 || W <= 0 || !(bits == 8 || bits == 64) || (uint64_t)n * (uint64_t)W * (uint64_t)(bits / 8) > P->bytes) return nullptr;
    DevSync& S = *sync_of(P->dev);
    const Sig* C = nullptr;
    {
        std::lock_guard<std::mutex> g(S.mu);
        for (auto& x : S.callers) if (x.s == (hipStream_t)caller) C = &x;
    }
    if (!C || !C->p) return nullptr;   // the counter wait only: the tag is a mark of the caller's counter
    Row* r = nullptr;
    {
        std::lock_guard<std::mutex> g(P->mu);
        for (size_t i = 0; i < P->free.size() && !r; i++) {
            Row* x = P->free[i];
            if (!x->caller || __atomic_load_n((const uint64_t*)x->caller->p, __ATOMIC_ACQUIRE) >= x->tag) {
                r = x;
                P->free.erase(P->free.begin() + (std::ptrdiff_t)i);
            }
        }
    }
    if (!r) return nullptr;
    r->caller = C;
    r->shape[0] = n; r->shape[1] = W;
    DLTensorV& t = r->mt.dl_tensor;
    t.data = r->ptr; t.device = DLDeviceV{DL_ROCM, P->dev}; t.ndim = 2;
    t.dtype = DLDataTypeV{(uint8_t)(bits == 8 ? DL_UINT : DL_INT), (uint8_t)bits, 1};
    t.shape = r->shape; t.strides = nullptr; t.byte_offset = 0;
    r->mt.manager_ctx = r;
    r->mt.deleter = row_deleter;
    return &r->mt;
}

extern "C" int32_t pv_rows_count(const void* pool, int32_t* total, int32_t* free_rows) {
    RowPool* P = (RowPool*)pool;
    if (!P) return PV_EARG;
    std::lock_guard<std::mutex> g(P->mu);
    if (total) *total = (int32_t)P->all.size();
    if (free_rows) *free_rows = (int32_t)P->free.size();
    return PV_OK;
}

namespace {
// FASTA bytes [f0, f0 + nf) of one assembly, laid out from its decoded base stream: per record '>' + header + '\n',
// then the bases in lines of lw, each followed by '\n' (the reference's Core::fasta layout, csrc/pv_core.cpp:138-159).
// rec: per record i64 {FASTA offset, header offset in hdrs, header length, length, base-stream offset, line width},
// in file order; `bases` holds stream positions [b0, b0 + nb). 16 output bytes per thread, stored as one 16-byte write.
__global__ void __launch_bounds__(256) fasta_layout_kernel(const uint8_t* __restrict__ bases, uint64_t b0, uint64_t nb,
                                                           const int64_t* __restrict__ rec, int32_t nrec, const uint8_t* __restrict__ hdrs,
                                                           uint64_t f0, uint64_t nf, uint8_t* __restrict__ out) {
    const uint64_t i0 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
    if (i0 >= nf) return;
    const uint64_t f = f0 + i0;
    int32_t lo = 0, hi = nrec - 1;                  // last record starting at or before f
    while (lo < hi) { const int32_t m = (lo + hi + 1) / 2; if ((uint64_t)rec[6 * m] <= f) lo = m; else hi = m - 1; }
    int32_t r = lo;
    const int64_t* R = rec + 6 * r;
    uint64_t next = r + 1 < nrec ? (uint64_t)rec[6 * (r + 1)] : ~0ull;
    uint8_t v[16];
    for (int k = 0; k < 16; k++) {
        const uint64_t x = f + k;
        if (i0 + k >= nf) { v[k] = 0; continue; }
        while (x >= next) { r++; R = rec + 6 * r; next = r + 1 < nrec ? (uint64_t)rec[6 * (r + 1)] : ~0ull; }
        const uint64_t rel = x - (uint64_t)R[0], hl = (uint64_t)R[2];
        uint8_t c;
        if (rel == 0) c = '>';
        else if (rel <= hl) c = hdrs[R[1] + rel - 1];
        else if (rel == hl + 1) c = '\n';
        else {
            const uint64_t q = rel - hl - 2, lw = (uint64_t)R[5], line = q / (lw + 1), col = q - line * (lw + 1);
            const uint64_t len = (uint64_t)R[3], llen = min(lw, len - line * lw);
            if (col < llen) {
                const uint64_t b = (uint64_t)R[4] + line * lw + col;
                c = (b >= b0 && b - b0 < nb) ? bases[b - b0] : 0;
            } else c = '\n';
        }
        v[k] = c;
    }
    if (i0 + 16 <= nf && (((uintptr_t)(out + i0)) & 15) == 0) {
        uint4 w;
        memcpy(&w, v, 16);
        *(uint4*)(out + i0) = w;
    } else {
        for (int k = 0; k < 16 && i0 + k < nf; k++) out[i0 + k] = v[k];
    }
}
}  // namespace

extern "C" int32_t pv_fasta_layout_hip(const uint8_t* bases, uint64_t b0, uint64_t nb, const int64_t* rec, int32_t nrec, const uint8_t* hdrs,
                                       uint64_t f0, uint64_t nf, uint8_t* out, void* stream, char* err, size_t errcap) {
    if (nf == 0) return PV_OK;
    if (!rec || nrec <= 0 || !out || (nb && !bases)) { seterr(err, errcap, "null argument"); return PV_EARG; }
    const uint64_t threads = (nf + 15) / 16, blocks = (threads + 255) / 256;
    if (blocks >= (1ull << 31)) { seterr(err, errcap, "range too large"); return PV_EARG; }
    hipLaunchKernelGGL(fasta_layout_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, bases, b0, nb, rec, nrec, hdrs, f0, nf, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    return PV_OK;
}
