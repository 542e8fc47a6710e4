// pv_codec.h - refrel3 v1 entropy grammar: constants and small pure functions shared by the host (archive reader,
// GPU model-table builder) and the HIP decode kernels.
//
// Grammar restated from the reference's codec (csrc/refrel3.h:24-62 contexts / buckets / classes, :68-91 rANS,
// :94-109 diagonals, :114-160 block grammar) and FORMAT.md sections 2-4. The context numbering, the alphabets, the
// bucket code and the diagonal arithmetic are part of the archive format, so they are necessarily the same values;
// the code around them is this build's own.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define PV_HD __host__ __device__
#else
#define PV_HD
#endif

namespace pvc {

// ---- contexts (refrel3.h:24, :29-41)
enum : int { C_LL = 0, C_LITR = 4, C_LIT2 = 14, C_KIND = 31, C_DELTA = 47, C_REPK = 49, C_REPD = 50, C_DIR = 51, C_SELF = 52,
             C_LEN = 53, C_FLIPK = 59, C_FLIPD = 60, NCTX = 61 };
enum : int { K_CONT = 0, K_DELTA = 1, K_REP = 2, K_ABS = 3, K_SELF = 4, K_FLIP = 5 };
static constexpr int BIG_ALPHA = 104;              // bucketed values: 16 small + 4 per octave
static constexpr uint32_t PROB_BITS = 12, M = 1u << PROB_BITS;   // frequencies sum to 4096 per context (or all 0)
static constexpr uint32_t RANS_L = 1u << 16;       // rANS state lives in [2^16, 2^24)
static constexpr uint32_t MIN_LEN = 12;            // copy length offset (refrel_format.h:31)

PV_HD constexpr int alpha_of(int c) {
    return (c < C_LITR) ? BIG_ALPHA : (c < C_DELTA) ? 6 : (c < C_REPK) ? BIG_ALPHA : (c == C_REPK) ? 3 : (c == C_REPD) ? BIG_ALPHA
         : (c == C_DIR) ? 2 : (c == C_SELF) ? BIG_ALPHA : (c < C_FLIPK) ? BIG_ALPHA : (c == C_FLIPK) ? 4 : BIG_ALPHA;
}

// ---- GPU model table (per assembly, derived at open from the archive's frequencies; 10240 bytes)
// Every context keeps only its cumulative frequencies; a symbol is the number of boundaries cum[1..alpha-1] that are
// <= the slot (cum is non-decreasing, so this equals the reference's sym[] lookup, refrel3.h:77, built by
// pv_v1.h:56-58), and its frequency is cum[s+1] - cum[s] (0 = a symbol from an all-zero context: decode failure).
//  small contexts (alphabet <= 6): 8 x u16 = cum[0..7], entries past the alphabet repeat the context total
//  big contexts (alphabet 104):   112 x u16 = cum[0..104], then padding
static constexpr int NSMALL = 46, NBIG = 15, SMALL_ROW = 8, BIG_ROW = 112;
static constexpr int GTAB_BYTES = 10240;
static constexpr int SMALL_BYTES = NSMALL * SMALL_ROW * 2;   // 736
//  literal-pair section at PAIR_OFF: for the 16 order-2 literal contexts r (LIT2 0..15) and the 16 symbol pairs
//  l = 4 s1 + s2 (A/C/G/T each), two u32 (lo | (freq - 4096) << 16, the high half a signed 16-bit number): symbol s1
//  in context r, then symbol s2 in the context that follows s1, ((r & 3) * 4 + s1). Entry (r, l) at PAIR_OFF + 8 (16 r + l).
static constexpr int PAIR_OFF = 4096, PAIR_BYTES = 16 * 16 * 8;
//  bucket entries of the big contexts at DIRECT_OFF, for the one-lane-per-block decoder: for big row k (0..14) and slot
//  bucket j (0..DIRECT_NB-1, DIRECT_W slots each) one u64 at DIRECT_OFF + 8 (DIRECT_NB k + j): s0 = the symbol whose
//  range holds the bucket's first slot (bits 0-6; DIRECT_NONE for an all-zero row), lo = cum[s0] (bits 7-18) and
//  e_i = cum[s0 + i] - 1 for i = 1, 2, 3 (bits 19-30, 31-42, 43-54; 4095 past the alphabet). A slot <= e_3 has symbol
//  s0 + (slot > e_1) + (slot > e_2) and its range [lo or e_i + 1, e_{i+1}] from the entry alone (one load); a larger
//  slot continues on the row from s0 + 3 (cum non-decreasing, so empty symbols between are passed over correctly).
static constexpr int DIRECT_NB = 32, DIRECT_W = (int)M / DIRECT_NB, DIRECT_NONE = 127;
static constexpr int DIRECT_OFF = PAIR_OFF + PAIR_BYTES, DIRECT_BYTES = NBIG * DIRECT_NB * 8;
static_assert(SMALL_BYTES + NBIG * BIG_ROW * 2 <= PAIR_OFF && DIRECT_OFF + DIRECT_BYTES <= GTAB_BYTES && GTAB_BYTES % 256 == 0, "gtab layout");
// u16 offset of context c's row inside the table
PV_HD constexpr int row_of(int c) {
    // small rows in context order, big rows after them in context order
    return alpha_of(c) != BIG_ALPHA
        ? SMALL_ROW * ((c < C_DELTA) ? (c - C_LITR) : (c == C_REPK) ? 43 : (c == C_DIR) ? 44 : 45)
        : SMALL_BYTES / 2 + BIG_ROW * ((c < C_LITR) ? c : (c < C_REPK) ? 4 + (c - C_DELTA) : (c == C_REPD) ? 6 : (c == C_SELF) ? 7
                                                       : (c < C_FLIPK) ? 8 + (c - C_LEN) : 14);
}

// ---- buckets (refrel3.h:45-60)
PV_HD constexpr uint32_t nbits_of(uint32_t s) { return s < 16 ? 0 : (s - 16) / 4 + 2; }
PV_HD constexpr uint64_t unbucket(uint32_t s, uint64_t extra) {
    return s < 16 ? (uint64_t)s : ((1ull << ((s - 16) / 4 + 4)) | ((uint64_t)((s - 16) & 3) << ((s - 16) / 4 + 2)) | extra);
}
// ---- classes (refrel3.h:61-63)
PV_HD constexpr int llc(uint64_t ll) { return ll == 0 ? 0 : ll == 1 ? 1 : ll <= 8 ? 2 : 3; }
PV_HD constexpr int kclass(int k) { return k < 0 ? 0 : k == K_CONT ? 1 : (k == K_DELTA || k == K_REP || k == K_FLIP) ? 2 : 3; }
// reference base code: A0 C1 G2 T3, N and every other byte 4 (refrel3.h:63,108 folded)
PV_HD constexpr int base4(uint8_t b) { return b == 'A' ? 0 : b == 'C' ? 1 : b == 'G' ? 2 : b == 'T' ? 3 : 4; }
// upper-case complement; other bytes unchanged (refrel_format.h:75)
PV_HD constexpr uint8_t comp(uint8_t b) { return b == 'A' ? 'T' : b == 'C' ? 'G' : b == 'G' ? 'C' : b == 'T' ? 'A' : b; }
// complement keeping case (pv_v1.h:74-75) and the token code (pv_v1.h:76)
PV_HD constexpr uint8_t comp_case(uint8_t b) {
    return b == 'A' ? 'T' : b == 'C' ? 'G' : b == 'G' ? 'C' : b == 'T' ? 'A' : b == 'a' ? 't' : b == 'c' ? 'g' : b == 'g' ? 'c' : b == 't' ? 'a' : b;
}
PV_HD constexpr uint8_t token(uint8_t b) {
    return (b | 0x20) == 'a' ? 0 : (b | 0x20) == 'c' ? 1 : (b | 0x20) == 'g' ? 2 : (b | 0x20) == 't' ? 3 : 4;
}
PV_HD constexpr int64_t unzigzag(uint64_t z) { return (int64_t)(z >> 1) ^ -(int64_t)(z & 1); }

// ---- diagonals (refrel3.h:94-102): c is kept as a two's-complement 64-bit value
PV_HD constexpr int64_t diag_expect(int64_t c, uint32_t dir, uint32_t o, uint64_t L) { return dir ? c - (int64_t)o - (int64_t)L + 1 : c + (int64_t)o; }
PV_HD constexpr int64_t diag_locus(int64_t c, uint32_t dir, uint32_t o) { return dir ? c - (int64_t)o : c + (int64_t)o; }
PV_HD constexpr int64_t diag_of(uint32_t dir, uint64_t p, uint32_t o, uint64_t L) { return dir ? (int64_t)p + (int64_t)L - 1 + (int64_t)o : (int64_t)p - (int64_t)o; }

}  // namespace pvc
