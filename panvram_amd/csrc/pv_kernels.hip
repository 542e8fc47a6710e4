// pv_kernels.hip - refrel3 v1 window decode on MI355X (gfx950).
//
// One 64-lane wavefront (one workgroup) per (window, covering block) slot:
//   1. stage into LDS, all lanes in parallel: the assembly's GPU model table (4 KB of cumulative frequencies), the
//      block's rANS payload, and the reference span the block's start diagonal predicts (plus a margin);
//   2. decode the block's symbol stream - the serial part - with every lane executing the same (wave-uniform) control
//      flow: a symbol of a 6-letter context is found by comparing the slot against the context's five boundaries, a
//      symbol of a 104-letter context by one compare per lane and two ballots; literals go straight into the LDS
//      block buffer, copies into an LDS op list;
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
#include <hip/hip_runtime.h>

#include "../../include/panvram_amd.h"
#include "pv_codec.h"

#include <stdio.h>

namespace {

constexpr int WAVE = 64;
constexpr uint32_t RMARGIN = 256;        // reference bytes staged on each side of the start diagonal's span

template <int Q> struct Cfg {
    static constexpr uint32_t PAYCAP = Q < 8192 ? 2 * Q : 8192;      // payload bytes staged in LDS (rest read from HBM)
    static constexpr uint32_t REFW = Q + 2 * RMARGIN + 32;           // staged reference span (+ alignment slack)
    static constexpr uint32_t MAXCOPY = Q / pvc::MIN_LEN + 1;        // copies per block: each >= 12 bases
};

template <int Q> struct __align__(16) Lds {
    uint8_t blk[Q];                                   // the block, upper case
    uint8_t refw[Cfg<Q>::REFW];                       // reference [wbase, wbase + REFW)
    uint8_t pay[Cfg<Q>::PAYCAP + 32];                 // payload, from its 16-byte aligned base
    uint16_t tab[pvc::GTAB_BYTES / 2];                // model table
    uint32_t ops[Cfg<Q>::MAXCOPY][2];                 // copy ops: src, dst | len << 15 | kind << 30
    uint32_t lower[Q / 32];                           // lower-case bitmask of the block
};

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x; }   // one wavefront per workgroup
__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// all lanes copy 16-byte aligned chunks covering [g, g + len) into dst (16-byte aligned), at most cap bytes.
// Returns g's offset inside dst. Source arrays carry >= 16 bytes of padding past their end.
__device__ __forceinline__ uint32_t stage(uint8_t* dst, const uint8_t* g, uint32_t len, uint32_t cap) {
    const uint4* a = (const uint4*)((uintptr_t)g & ~(uintptr_t)15);
    const uint32_t mis = (uint32_t)((uintptr_t)g & 15);
    uint32_t nch = (mis + len + 15) / 16; if (nch > cap / 16) nch = cap / 16;
    uint4* d = (uint4*)dst;
    const uint32_t l = lane_id();
    for (uint32_t c = l; c < nch; c += 4 * WAVE) {
        uint4 v0, v1, v2, v3;
        const bool p1 = c + WAVE < nch, p2 = c + 2 * WAVE < nch, p3 = c + 3 * WAVE < nch;
        v0 = a[c];
        if (p1) v1 = a[c + WAVE];
        if (p2) v2 = a[c + 2 * WAVE];
        if (p3) v3 = a[c + 3 * WAVE];
        d[c] = v0;
        if (p1) d[c + WAVE] = v1;
        if (p2) d[c + 2 * WAVE] = v2;
        if (p3) d[c + 3 * WAVE] = v3;
    }
    return mis;
}

// ---- rANS decoder state (wave-uniform)
struct Dec {
    uint32_t x;          // state
    uint32_t p, n;       // next payload byte, payload length
    uint32_t mis;        // payload offset inside the LDS copy
    uint32_t cap;        // bytes available in the LDS copy (from the payload start)
    const uint8_t* g;    // payload in HBM
    bool bad;
};

template <int Q> __device__ __forceinline__ uint32_t pay_byte(const Lds<Q>& S, const Dec& d, uint32_t i) {
    return i < d.cap ? S.pay[d.mis + i] : d.g[i];
}
template <int Q> __device__ __forceinline__ void renorm(const Lds<Q>& S, Dec& d) {
    while (d.x < pvc::RANS_L) {
        if (d.p >= d.n) { d.bad = true; return; }
        d.x = (d.x << 8) | pay_byte(S, d, d.p); d.p++;
    }
}
// symbol of a context with <= 6 letters (row = 8 cumulative frequencies in LDS)
template <int Q> __device__ __forceinline__ uint32_t sym_small(const Lds<Q>& S, Dec& d, int row) {
    const uint4 r = *(const uint4*)&S.tab[row];
    const uint32_t slot = d.x & (pvc::M - 1);
    const uint32_t c1 = r.x >> 16, c2 = r.y & 0xFFFF, c3 = r.y >> 16, c4 = r.z & 0xFFFF, c5 = r.z >> 16, c6 = r.w & 0xFFFF;
    const uint32_t s = (c1 <= slot) + (c2 <= slot) + (c3 <= slot) + (c4 <= slot) + (c5 <= slot);
    uint32_t lo, hi;
    switch (s) {
        case 0: lo = 0; hi = c1; break;
        case 1: lo = c1; hi = c2; break;
        case 2: lo = c2; hi = c3; break;
        case 3: lo = c3; hi = c4; break;
        case 4: lo = c4; hi = c5; break;
        default: lo = c5; hi = c6; break;
    }
    const uint32_t f = hi - lo;
    if (!f) { d.bad = true; return s; }
    d.x = f * (d.x >> pvc::PROB_BITS) + slot - lo;
    renorm(S, d);
    return s;
}
// symbol of a 104-letter context: lane l compares cum[l+1] and cum[l+65]; the symbol is the number of boundaries <= slot
template <int Q> __device__ __forceinline__ uint32_t sym_big(const Lds<Q>& S, Dec& d, int row) {
    const uint32_t l = lane_id();
    const uint16_t* r = &S.tab[row];
    const uint32_t a = r[l + 1];
    const uint32_t b = (l + 65 <= (uint32_t)pvc::BIG_ALPHA) ? (uint32_t)r[l + 65] : 0xFFFFu;
    const uint32_t slot = d.x & (pvc::M - 1);
    const uint64_t m0 = __ballot(a <= slot && l + 1 < (uint32_t)pvc::BIG_ALPHA);
    const uint64_t m1 = __ballot(b <= slot && l + 65 < (uint32_t)pvc::BIG_ALPHA);
    const uint32_t s = (uint32_t)(__popcll(m0) + __popcll(m1));
    const uint32_t lo = s == 0 ? 0u : (s <= 64 ? (uint32_t)__builtin_amdgcn_readlane((int)a, (int)(s - 1)) : (uint32_t)__builtin_amdgcn_readlane((int)b, (int)(s - 65)));
    const uint32_t hi = s + 1 <= 64 ? (uint32_t)__builtin_amdgcn_readlane((int)a, (int)s) : (uint32_t)__builtin_amdgcn_readlane((int)b, (int)(s - 64));
    const uint32_t f = hi - lo;
    if (!f) { d.bad = true; return s; }
    d.x = f * (d.x >> pvc::PROB_BITS) + slot - lo;
    renorm(S, d);
    return s;
}
// raw bits, <= 16 per step, low chunk first (csrc/refrel3.h:83-90)
template <int Q> __device__ __forceinline__ uint64_t draw(const Lds<Q>& S, Dec& d, uint32_t nb) {
    uint64_t v = 0; uint32_t sh = 0;
    while (nb && !d.bad) {
        const uint32_t k = nb > 16 ? 16 : nb;
        const uint32_t b = d.x & ((1u << k) - 1); d.x >>= k;
        renorm(S, d);
        v |= (uint64_t)b << sh; sh += k; nb -= k;
    }
    return v;
}
template <int Q> __device__ __forceinline__ uint64_t dval_big(const Lds<Q>& S, Dec& d, int row) {
    const uint32_t s = sym_big(S, d, row);
    if (d.bad) return 0;
    return pvc::unbucket(s, draw(S, d, pvc::nbits_of(s)));
}

constexpr int SMALL_ROW_LITR = pvc::row_of(pvc::C_LITR), SMALL_ROW_LIT2 = pvc::row_of(pvc::C_LIT2), SMALL_ROW_KIND = pvc::row_of(pvc::C_KIND);
constexpr int ROW_REPK = pvc::row_of(pvc::C_REPK), ROW_DIR = pvc::row_of(pvc::C_DIR), ROW_FLIPK = pvc::row_of(pvc::C_FLIPK);
constexpr int ROW_LL = pvc::row_of(pvc::C_LL), ROW_DELTA = pvc::row_of(pvc::C_DELTA), ROW_REPD = pvc::row_of(pvc::C_REPD);
constexpr int ROW_SELF = pvc::row_of(pvc::C_SELF), ROW_LEN = pvc::row_of(pvc::C_LEN), ROW_FLIPD = pvc::row_of(pvc::C_FLIPD);
static_assert(pvc::row_of(pvc::C_LITR + 9) == SMALL_ROW_LITR + 9 * pvc::SMALL_ROW, "small rows contiguous");
static_assert(pvc::row_of(pvc::C_KIND + 15) == SMALL_ROW_KIND + 15 * pvc::SMALL_ROW, "small rows contiguous");
static_assert(pvc::row_of(pvc::C_LL + 3) == ROW_LL + 3 * pvc::BIG_ROW, "big rows contiguous");
static_assert(pvc::row_of(pvc::C_DELTA + 1) == ROW_DELTA + pvc::BIG_ROW, "big rows contiguous");
static_assert(pvc::row_of(pvc::C_LEN + 5) == ROW_LEN + 5 * pvc::BIG_ROW, "big rows contiguous");

// reference view: a staged span in LDS, HBM elsewhere
struct RefView { const uint8_t* g; uint64_t n; int64_t wbase; uint32_t wlen; };
template <int Q> __device__ __forceinline__ uint8_t ref_at(const Lds<Q>& S, const RefView& R, uint64_t q) {
    const uint64_t k = q - (uint64_t)R.wbase;
    return k < R.wlen ? S.refw[k] : R.g[q];
}

struct Diag { int64_t c; uint32_t dir; };

// decode one block into S.blk (literals) and S.ops (copies). Returns the number of copy ops, or -1 on failure
// (csrc/refrel3.h:114-160; every failure condition of the reference fails here too).
template <int Q> __device__ int decode_block(Lds<Q>& S, Dec& d, const RefView& R, uint32_t blen, Diag start) {
    Diag cache[4]; int nc = 1; cache[0] = start;
    int prevk = -1; uint32_t o = 0; int nops = 0;
    while (o < blen) {
        const uint64_t ll = dval_big(S, d, ROW_LL + pvc::BIG_ROW * pvc::kclass(prevk));
        if (d.bad || ll > blen - o) return -1;
        if (ll) {
            uint32_t p1 = 16, p2 = 16;
            for (uint32_t j = 0; j < (uint32_t)ll; j++) {
                int row;
                if (ll <= 8) {
                    const int64_t q = pvc::diag_locus(cache[0].c, cache[0].dir, o + j);
                    int rb = 4;
                    if (q >= 0 && (uint64_t)q < R.n) { uint8_t b = ref_at(S, R, (uint64_t)q); if (cache[0].dir) b = pvc::comp(b); rb = pvc::base4(b); }
                    row = SMALL_ROW_LITR + pvc::SMALL_ROW * (rb * 2 + (j == 0 ? 1 : 0));
                } else {
                    const int cx = p1 == 16 ? 16 : (int)(p2 == 16 ? p1 : p2 * 4 + p1) % 16;
                    row = SMALL_ROW_LIT2 + pvc::SMALL_ROW * cx;
                }
                const uint32_t s = sym_small(S, d, row);
                if (d.bad) return -1;
                uint8_t byte;
                if (s < 5) byte = (uint8_t)(s == 0 ? 'A' : s == 1 ? 'C' : s == 2 ? 'G' : s == 3 ? 'T' : 'N');
                else { byte = (uint8_t)draw(S, d, 8); if (d.bad) return -1; }
                S.blk[o + j] = byte;
                p2 = p1; p1 = s < 4 ? s : 0;
            }
            o += (uint32_t)ll;
        }
        if (o == blen) break;
        const int kind = (int)sym_small(S, d, SMALL_ROW_KIND + pvc::SMALL_ROW * (pvc::llc(ll) * 4 + pvc::kclass(prevk)));
        if (d.bad) return -1;
        uint64_t p = 0; uint32_t dir = 0; int ki = 0; int64_t dd = 0; uint64_t dist = 0;
        if (kind == pvc::K_CONT) {
        } else if (kind == pvc::K_DELTA) {
            dd = pvc::unzigzag(dval_big(S, d, ROW_DELTA + pvc::BIG_ROW * (ll == 0 ? 0 : 1)));
        } else if (kind == pvc::K_REP) {
            ki = 1 + (int)sym_small(S, d, ROW_REPK);
            if (d.bad) return -1;
            dd = pvc::unzigzag(dval_big(S, d, ROW_REPD));
            if (ki >= nc) return -1;
        } else if (kind == pvc::K_ABS) {
            dir = sym_small(S, d, ROW_DIR);
            if (d.bad) return -1;
            p = draw(S, d, 32);
        } else if (kind == pvc::K_SELF) {
            dist = dval_big(S, d, ROW_SELF);
        } else if (kind == pvc::K_FLIP) {
            ki = (int)sym_small(S, d, ROW_FLIPK);
            if (d.bad) return -1;
            dd = pvc::unzigzag(dval_big(S, d, ROW_FLIPD));
            if (ki >= nc) return -1;
        } else {
            return -1;
        }
        if (d.bad) return -1;
        const uint64_t L = dval_big(S, d, ROW_LEN + pvc::BIG_ROW * kind) + pvc::MIN_LEN;
        if (d.bad || L > blen - o) return -1;
        uint32_t okind; uint64_t osrc;
        if (kind == pvc::K_SELF) {
            if (dist == 0 || dist > o) return -1;
            okind = 2; osrc = o - dist;
        } else {
            if (kind == pvc::K_FLIP) {
                const Diag g = cache[ki]; dir = g.dir ^ 1;
                const int64_t e = pvc::diag_locus(g.c, g.dir, o) + dd; if (e < 0) return -1; p = (uint64_t)e;
            } else if (kind != pvc::K_ABS) {
                const Diag g = cache[kind == pvc::K_REP ? ki : 0]; dir = g.dir;
                const int64_t e = pvc::diag_expect(g.c, g.dir, o, L) + dd; if (e < 0) return -1; p = (uint64_t)e;
            }
            if (p > R.n || L > R.n - p) return -1;
            okind = dir ? 3 : 1; osrc = p;
            // move-to-front diagonal cache of <= 4 (csrc/refrel3.h:98-102)
            const Diag ng = {pvc::diag_of(dir, p, o, L), dir};
            int j = 0; while (j < nc && !(cache[j].c == ng.c && cache[j].dir == ng.dir)) j++;
            if (j == nc) { if (nc < 4) nc++; j = nc - 1; }
            for (; j > 0; j--) cache[j] = cache[j - 1];
            cache[0] = ng;
        }
        if (nops >= (int)Cfg<Q>::MAXCOPY) return -1;   // cannot happen: copies are >= 12 bases
        S.ops[nops][0] = (uint32_t)osrc;
        S.ops[nops][1] = o | ((uint32_t)L << 15) | (okind << 30);
        nops++;
        o += (uint32_t)L; prevk = kind;
    }
    if (d.bad || d.x != pvc::RANS_L || d.p != d.n) return -1;
    return nops;
}

template <int Q>
__global__ void __launch_bounds__(WAVE) windows_kernel(pv_dev_cohort D, const int64_t* __restrict__ wasm, const int64_t* __restrict__ wstart,
                                                     uint32_t W, uint32_t bpw, const uint8_t* __restrict__ rcm, int tokens, int apply_case,
                                                     uint8_t* __restrict__ out, int* __restrict__ status) {
    __shared__ Lds<Q> S;
    const uint32_t l = lane_id();
    const uint64_t w = blockIdx.x / bpw; const uint32_t j = blockIdx.x % bpw;
    const int64_t a = wasm[w];
    if (a < 0 || a >= D.nasm) { if (l == 0 && j == 0) atomicOr(status, PV_ST_RANGE); return; }
    const int64_t* ar = D.asm_rec + 8 * a;
    const int64_t pay_base = ar[0], blk_base = ar[1], nbases = ar[2], low_base = ar[3], low_cnt = ar[4];
    const int64_t s0 = wstart[w];
    if (s0 < 0 || (uint64_t)s0 + W > (uint64_t)nbases) { if (l == 0 && j == 0) atomicOr(status, PV_ST_RANGE); return; }
    const uint64_t s = (uint64_t)s0;
    const uint64_t b0 = s / Q, b1 = (s + W - 1) / Q, b = b0 + j;
    if (b > b1) return;
    const uint64_t bst = b * Q;
    const uint32_t blen = (uint32_t)min((uint64_t)Q, (uint64_t)nbases - bst);
    const uint64_t bb = (uint64_t)blk_base + b;
    const uint32_t poff = D.off[bb], plen = D.off[bb + 1] - poff;
    const int64_t stv = D.st[bb];
    const Diag g0 = {stv >> 1, (uint32_t)(stv & 1)};
    const uint8_t* gpay = D.P + pay_base + poff;

    // 1. stage table, payload and the reference span of the start diagonal
    stage((uint8_t*)S.tab, D.tab + (uint64_t)a * pvc::GTAB_BYTES, pvc::GTAB_BYTES, pvc::GTAB_BYTES);
    Dec d; d.p = 0; d.n = plen; d.g = gpay; d.bad = false;
    d.mis = stage(S.pay, gpay, plen, Cfg<Q>::PAYCAP + 16);
    d.cap = min(plen, Cfg<Q>::PAYCAP + 16 - d.mis);
    RefView R; R.g = D.ref; R.n = D.ref_n; R.wbase = 0; R.wlen = 0;
    {
        const int64_t lo = g0.dir ? g0.c - (int64_t)blen + 1 : g0.c, hi = lo + (int64_t)blen;   // span [lo, hi)
        int64_t wl = lo - (int64_t)RMARGIN, wh = hi + (int64_t)RMARGIN;
        if (wl < 0) wl = 0;
        if (wh > (int64_t)D.ref_n) wh = (int64_t)D.ref_n;
        if (wl < wh) {
            const uint32_t mis = stage(S.refw, D.ref + wl, (uint32_t)(wh - wl), Cfg<Q>::REFW);
            R.wbase = wl - (int64_t)mis;
            R.wlen = min((uint32_t)(wh - wl) + mis, (uint32_t)Cfg<Q>::REFW);
        }
    }
    __syncthreads();

    // 2. decode
    int nops;
    if (plen < 3) nops = -1;
    else {
        d.x = pay_byte(S, d, 0) | (pay_byte(S, d, 1) << 8) | (pay_byte(S, d, 2) << 16); d.p = 3;
        nops = decode_block(S, d, R, blen, g0);
    }
    if (nops < 0) { if (l == 0) atomicOr(status, PV_ST_DECODE); return; }
    __syncthreads();

    // 3. replay the copies the window part [r0, r1) of this block needs
    const uint32_t r0 = (uint32_t)(max(s, bst) - bst), r1 = (uint32_t)(min(s + W, bst + blen) - bst);
    uint32_t need = r0;           // lowest block position still needed: self copies pull it down
    int klast = nops - 1;
    while (klast >= 0 && (S.ops[klast][1] & 0x7FFF) >= r1) klast--;
    int kfirst = klast + 1;
    for (int k = klast; k >= 0; k--) {
        const uint32_t w1 = S.ops[k][1], dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF;
        if (dst + len <= need) break;     // ops are in block order: every earlier one ends before `need` too
        kfirst = k;
        if ((w1 >> 30) == 2) { const uint32_t src = S.ops[k][0]; if (src < need) need = src; }
    }
    for (int k = kfirst; k <= klast; k++) {
        const uint32_t src = S.ops[k][0], w1 = S.ops[k][1], dst = w1 & 0x7FFF, len = (w1 >> 15) & 0x7FFF, kind = w1 >> 30;
        const uint32_t i0 = need > dst ? need - dst : 0, i1 = min(len, r1 - dst);
        if (kind == 1) {
            for (uint32_t i = i0 + l; i < i1; i += WAVE) S.blk[dst + i] = ref_at(S, R, (uint64_t)src + i);
        } else if (kind == 3) {
            const uint64_t top = (uint64_t)src + len - 1;
            for (uint32_t i = i0 + l; i < i1; i += WAVE) S.blk[dst + i] = pvc::comp(ref_at(S, R, top - i));
        } else {
            const uint32_t dist = dst - src;
            for (uint32_t i = i0 + l; i < i1; i += WAVE) S.blk[dst + i] = S.blk[src + (i % dist)];
        }
        __syncthreads();
    }

    // 4. lower-case bitmask of [r0, r1), then the write-out with the transforms
    const bool do_case = apply_case && !tokens && low_cnt > 0;
    if (do_case) {
        const uint32_t wd0 = r0 / 32, wd1 = (r1 + 31) / 32;
        uint32_t acc[Q / 32 / WAVE > 0 ? Q / 32 / WAVE : 1];
        constexpr int NW = Q / 32 / WAVE > 0 ? Q / 32 / WAVE : 1;
        for (int k = 0; k < NW; k++) acc[k] = 0;
        const int64_t* ls = D.low_s + low_base; const int64_t* ln = D.low_l + low_base;
        const uint64_t x0 = bst + r0, x1 = bst + r1;
        for (int64_t r = D.run0[bb]; r < low_cnt; r += WAVE) {
            const int64_t rr = r + l;
            int64_t rs = INT64_MAX, re = INT64_MAX;
            if (rr < low_cnt) { rs = ls[rr]; re = rs + ln[rr]; }
            // runs are sorted: stop once one starts at or after the window part's end
            const uint64_t stop = __ballot(rr < low_cnt && (uint64_t)rs >= x1);
            const uint64_t live = __ballot(rr < low_cnt && (uint64_t)rs < x1 && (uint64_t)re > x0);
            for (uint64_t m = live; m; m &= m - 1) {
                const int src_l = __ffsll((unsigned long long)m) - 1;
                const int64_t a0 = readlane64(rs, src_l), a1 = readlane64(re, src_l);
                const uint32_t q0 = (uint32_t)(max((uint64_t)a0, x0) - bst), q1 = (uint32_t)(min((uint64_t)a1, x1) - bst);
                for (int k = 0; k < NW; k++) {
                    const uint32_t wd = l + (uint32_t)k * WAVE, wb0 = wd * 32, wb1 = wb0 + 32;
                    if (wd < wd0 || wd >= wd1) continue;
                    const uint32_t lo = max(q0, wb0), hi = min(q1, wb1);
                    if (lo < hi) {
                        const uint32_t nbit = hi - lo;
                        const uint32_t mask = (nbit == 32 ? 0xFFFFFFFFu : ((1u << nbit) - 1)) << (lo - wb0);
                        acc[k] |= mask;
                    }
                }
            }
            if (stop) break;
        }
        for (int k = 0; k < NW; k++) { const uint32_t wd = l + (uint32_t)k * WAVE; if (wd < Q / 32) S.lower[wd] = acc[k]; }
        __syncthreads();
    }
    const bool rc = rcm && rcm[w];
    uint8_t* row = out + w * (uint64_t)W;
    for (uint32_t x = r0 + l; x < r1; x += WAVE) {
        uint8_t v = S.blk[x];
        if (do_case && ((S.lower[x >> 5] >> (x & 31)) & 1)) v |= 0x20;
        const uint64_t t = bst + x - s;
        uint64_t pos = t;
        if (rc) { v = pvc::comp_case(v); pos = (uint64_t)W - 1 - t; }
        if (tokens) v = pvc::token(v);
        row[pos] = v;
    }
}

void seterr(char* e, size_t cap, const char* m) { if (e && cap) snprintf(e, cap, "%s", m); }

template <int Q>
hipError_t launch(const pv_dev_cohort& D, const int64_t* wa, const int64_t* ws, uint32_t W, uint32_t bpw, uint64_t nslots, const uint8_t* rc,
                  int tokens, int apply_case, uint8_t* out, int32_t* status, hipStream_t st) {
    hipLaunchKernelGGL((windows_kernel<Q>), dim3((uint32_t)nslots), dim3(WAVE), 0, st, D, wa, ws, W, bpw, rc, tokens, apply_case, out, (int*)status);
    return hipGetLastError();
}

}  // namespace

extern "C" int32_t pv_windows_hip(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W, const uint8_t* rc,
                                  int32_t tokens, int32_t apply_case, uint8_t* out, int32_t* status, void* stream, char* err, size_t errcap) {
    if (!D || (!asm_idx && n) || (!start && n) || !status || (!out && n && W)) { seterr(err, errcap, "null argument"); return PV_EARG; }
    const uint32_t Q = D->Q;
    if (!(Q == 1024 || Q == 2048 || Q == 4096 || Q == 16384)) { seterr(err, errcap, "block size"); return PV_EARG; }
    if (W < 0 || W >= (1ll << 31)) { seterr(err, errcap, "W"); return PV_EARG; }
    if (n < 0) { seterr(err, errcap, "n"); return PV_EARG; }
    if (n == 0 || W == 0) return PV_OK;
    const uint64_t bpw = ((uint64_t)W + Q - 1) / Q + 1;
    if ((uint64_t)n * bpw >= (1ull << 31)) { seterr(err, errcap, "too many blocks in one call (windows x blocks per window >= 2^31)"); return PV_EARG; }
    const uint64_t nslots = (uint64_t)n * bpw;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    switch (Q) {
        case 1024: e = launch<1024>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, status, st); break;
        case 2048: e = launch<2048>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, status, st); break;
        case 4096: e = launch<4096>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, status, st); break;
        default: e = launch<16384>(*D, asm_idx, start, (uint32_t)W, (uint32_t)bpw, nslots, rc, tokens, apply_case, out, status, st); break;
    }
    if (e != hipSuccess) { seterr(err, errcap, hipGetErrorString(e)); return PV_EHIP; }
    return PV_OK;
}
