// cohortgen.cpp - synthetic pangenome cohorts for the tests and the benchmark: a reference FASTA (i.i.d. bases at a
// given GC, N runs, optional centromere-like N regions holding 171-bp satellite arrays, optional soft-mask runs) and
// haplotype assemblies derived from it by SNVs, indels and structural variants, each written as a refrel3 v1 archive.
//
// The generator knows every edit, so the encoder emits the copy events directly (no match search): a haplotype is a
// list of segments - reference copies (forward or reverse complement) and literal bases - and each block's events,
// symbols, model tables and rANS streams follow the format's grammar (reference FORMAT.md sections 1-4; the decoder
// semantics of csrc/refrel3.h:114-160 fix what the encoder must produce). Encoding is this build's own; archive
// bytes differ from the reference encoder's (which searches matches), the decoded bytes are what the tests pin:
// every archive's header carries the XXH3 of its source FASTA, of its base stream and of every block, computed here
// from the materialised haplotype, and the decoders must reproduce them.
//
// Test and benchmark infrastructure: nothing in panvram_amd/ uses it.
#include "../../panvram_amd/csrc/pv_codec.h"
#include "../../panvram_amd/csrc/pv_sha256.h"
#include "../../panvram_amd/csrc/pv_xxh3.h"

#include <dlfcn.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>
#include <chrono>
#include <cstdlib>

extern "C" {
size_t ZSTD_compress(void* dst, size_t cap, const void* src, size_t n, int level);
size_t ZSTD_compressBound(size_t n);
unsigned ZSTD_isError(size_t code);
}

namespace {

// phase timing on stderr when COHORTGEN_VERBOSE is set
double now_s() { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); }
void phase(const char* what, double t0) { static const bool v = getenv("COHORTGEN_VERBOSE") != nullptr; if (v) fprintf(stderr, "cohortgen %-28s %.2f s\n", what, now_s() - t0); }

// ------------------------------------------------------------------ RNG (splitmix64 seeding, xoshiro256**)
struct Rng {
    uint64_t s[4];
    static uint64_t sm(uint64_t& x) { uint64_t z = (x += 0x9E3779B97F4A7C15ull); z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull; z = (z ^ (z >> 27)) * 0x94D049BB133111EBull; return z ^ (z >> 31); }
    explicit Rng(uint64_t seed) { for (auto& v : s) v = sm(seed); }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() { const uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17; s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3]; s[2] ^= t; s[3] = rotl(s[3], 45); return r; }
    double uni() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
    uint64_t below(uint64_t n) { return n ? next() % n : 0; }
    uint64_t range(uint64_t lo, uint64_t hi) { return lo + below(hi - lo + 1); }           // inclusive
    uint64_t geom(double mean) { const double p = 1.0 / mean; return 1 + (uint64_t)std::floor(std::log(1.0 - uni()) / std::log(1.0 - p)); }  // >= 1
};
uint64_t mix(uint64_t a, uint64_t b) { uint64_t x = a * 0x9E3779B97F4A7C15ull ^ (b + 0x632BE59BD9B4E019ull); return Rng::sm(x); }

const uint8_t COMP_T[256] = {
#define C(x) (uint8_t)(x == 'A' ? 'T' : x == 'C' ? 'G' : x == 'G' ? 'C' : x == 'T' ? 'A' : x == 'a' ? 't' : x == 'c' ? 'g' : x == 'g' ? 'c' : x == 't' ? 'a' : x)
#define R4(b) C(b), C(b + 1), C(b + 2), C(b + 3)
#define R16(b) R4(b), R4(b + 4), R4(b + 8), R4(b + 12)
    R16(0), R16(16), R16(32), R16(48), R16(64), R16(80), R16(96), R16(112), R16(128), R16(144), R16(160), R16(176), R16(192), R16(208), R16(224), R16(240)
#undef R16
#undef R4
#undef C
};
inline uint8_t up(uint8_t c) { return (c >= 'a' && c <= 'z') ? (uint8_t)(c - 32) : c; }

// ------------------------------------------------------------------ parameters (filled by the Python wrapper)
struct RefParams {
    uint64_t seed;
    int32_t ncontigs; int32_t line_width;
    const uint64_t* lengths;
    double gc;
    int32_t n_runs; uint64_t n_run_min, n_run_max;        // N runs placed uniformly over the genome
    double centro_frac;                                     // per contig: an N region of this fraction (0 = none)
    uint64_t sat_min, sat_max; int32_t sat_monomer;         // satellite arrays inside the centromere region
    double mask_mean;                                       // soft-mask runs (alternating, geometric mean); 0 = none
    int32_t iupac_runs;                                     // runs of 1-4 segments of IUPAC codes (R, Y, K, ... N), each 1-5 long
    uint64_t n_run_at;                                      // > 0: a 64-base N run starting 32 bases before this position
};
struct AsmParams {
    uint64_t seed;
    int32_t n_asm, Q, line_width_a, line_width_b, block_hashes, threads, zstd_level;
    double snv_rate, indel_rate, indel_mean; uint32_t indel_max;
    int32_t sv_per_contig, sv_per_asm; uint64_t sv_min, sv_max;
    int32_t frag_min, frag_max;      // 0 = whole contigs; else each contig cut into [min, max] pieces
    double rc_piece;                 // probability a piece is stored reverse-complemented
    const char* prefix;              // archive names: <prefix><index>.<q>k.rr3
    double ins_odd;                  // probability that an inserted base is N or an IUPAC code (test cohorts; 0 = off)
};

struct Reference {
    std::vector<uint8_t> seq;                    // with case (soft mask)
    std::vector<uint64_t> off, len;              // contig offsets / lengths
    std::vector<std::string> names;
    bool has_lower = false;                      // soft mask present
};

// ------------------------------------------------------------------ reference
void make_reference(const RefParams& P, Reference& R, int threads) {
    uint64_t total = 0;
    for (int c = 0; c < P.ncontigs; c++) { R.off.push_back(total); R.len.push_back(P.lengths[c]); total += P.lengths[c]; R.names.push_back("chr" + std::to_string(c + 1)); }
    R.seq.resize(total);
    const uint64_t CH = 1 << 22, nch = (total + CH - 1) / CH;
    const uint32_t tg = (uint32_t)(P.gc / 2 * 65536), tc = (uint32_t)(P.gc * 65536), ta = (uint32_t)((P.gc + (1 - P.gc) / 2) * 65536);
    std::atomic<uint64_t> next{0}; std::vector<std::thread> th;
    for (int t = 0; t < threads; t++) th.emplace_back([&] {
        for (;;) {
            const uint64_t k = next.fetch_add(1); if (k >= nch) break;
            Rng r(mix(P.seed, k));
            const uint64_t a = k * CH, b = std::min(total, a + CH);
            for (uint64_t i = a; i < b; i += 4) {
                const uint64_t v = r.next();
                for (int j = 0; j < 4 && i + j < b; j++) {
                    const uint32_t u = (uint32_t)(v >> (16 * j)) & 0xFFFF;
                    R.seq[i + j] = u < tg ? 'G' : u < tc ? 'C' : u < ta ? 'A' : 'T';
                }
            }
        }
    });
    for (auto& x : th) x.join();
    Rng r(mix(P.seed, 0xC0FFEE));
    // centromere-like N regions with satellite arrays
    if (P.centro_frac > 0) {
        std::vector<uint8_t> mono(P.sat_monomer);
        for (auto& m : mono) m = "ACGT"[r.below(4)];
        for (int c = 0; c < P.ncontigs; c++) {
            const uint64_t L = R.len[c], reg = (uint64_t)(L * P.centro_frac);
            if (reg < 1000) continue;
            const uint64_t at = R.off[c] + L / 3;
            memset(&R.seq[at], 'N', reg);
            uint64_t x = at + reg / 10;
            while (P.sat_max && x < at + reg) {
                const uint64_t al = r.range(P.sat_min, P.sat_max);
                if (x + al > at + reg - reg / 10) break;
                for (uint64_t i = 0; i < al; i++) R.seq[x + i] = mono[i % P.sat_monomer];
                for (uint64_t i = r.geom(50.0) - 1; i < al; i += r.geom(50.0)) R.seq[x + i] = "ACGT"[r.below(4)];   // ~2 % divergence
                x += al + r.range(10000, 100000);
            }
        }
    }
    for (int k = 0; k < P.n_runs; k++) {
        const uint64_t l = r.range(P.n_run_min, P.n_run_max), p = r.below(total > l ? total - l : 1);
        memset(&R.seq[p], 'N', std::min(l, total - p));
    }
    static const char IUPAC[] = "RYKMSWBDHVN";
    for (int k = 0; k < P.iupac_runs && total > 64; k++) {
        uint64_t p = r.below(total - 64);
        const int segs = (int)r.range(1, 4);
        for (int g = 0; g < segs; g++) {
            const uint8_t b = (uint8_t)IUPAC[r.below(11)];
            for (uint64_t e = p + r.range(1, 5); p < e; p++) R.seq[p] = b;
        }
    }
    if (P.n_run_at >= 32 && P.n_run_at + 32 <= total) memset(&R.seq[P.n_run_at - 32], 'N', 64);
    if (P.mask_mean > 0) {
        R.has_lower = true;
        bool lower = r.below(2);
        for (uint64_t i = 0; i < total;) {
            const uint64_t l = std::min(r.geom(P.mask_mean), total - i);
            if (lower) for (uint64_t j = i; j < i + l; j++) R.seq[j] |= 0x20;   // 'N' -> 'n' as well
            lower = !lower; i += l;
        }
    }
}

bool write_fasta_ref(const Reference& R, int lw, const std::string& path) {
    FILE* f = fopen(path.c_str(), "wb"); if (!f) return false;
    std::vector<uint8_t> buf((1u << 24) + 4096); size_t w = 0;
    for (size_t c = 0; c < R.len.size(); c++) {
        const std::string h = ">" + R.names[c] + " synthetic\n";
        memcpy(&buf[w], h.data(), h.size()); w += h.size();
        const uint8_t* src = &R.seq[R.off[c]];
        for (uint64_t x = 0; x < R.len[c]; x += lw) {
            const uint64_t k = std::min<uint64_t>(lw, R.len[c] - x);
            memcpy(&buf[w], src + x, k); w += k; buf[w++] = '\n';
            if (w >= (1u << 24)) { fwrite(buf.data(), 1, w, f); w = 0; }
        }
    }
    fwrite(buf.data(), 1, w, f);
    return fclose(f) == 0;
}

// ------------------------------------------------------------------ haplotypes as segments
// A segment: `len` bases; ref >= 0: a copy of reference [ref, ref + len) (dir 0) or its reverse complement (dir 1);
// ref < 0: literal bases lit[lo, lo + len) (case kept).
struct Seg { uint64_t len; int64_t ref; uint32_t dir; uint64_t lo; };
struct Record { std::string hdr; uint32_t lw; std::vector<Seg> segs; uint64_t len; };

struct Hap {
    std::vector<Record> rec;
    std::vector<uint8_t> lit;
};

void push_copy(std::vector<Seg>& v, int64_t ref, uint64_t len) {
    if (!len) return;
    if (!v.empty() && v.back().ref >= 0 && v.back().dir == 0 && v.back().ref + (int64_t)v.back().len == ref) { v.back().len += len; return; }
    v.push_back({len, ref, 0, 0});
}
void push_lit(std::vector<Seg>& v, std::vector<uint8_t>& lit, const uint8_t* b, uint64_t len) {
    if (!len) return;
    if (!v.empty() && v.back().ref < 0 && v.back().lo + v.back().len == lit.size()) v.back().len += len;
    else v.push_back({len, -1, 0, lit.size()});
    lit.insert(lit.end(), b, b + len);
}

// one haplotype contig from reference contig c: SNVs, indels, SVs (sorted events applied left to right)
std::vector<Seg> mutate_contig(const Reference& R, int c, const AsmParams& P, Rng& r, int n_sv, std::vector<uint8_t>& lit) {
    struct Ev { uint64_t pos; int type; uint64_t len; };     // 0 snv, 1 ins, 2 del
    std::vector<Ev> ev;
    const uint64_t L = R.len[c], base = R.off[c];
    const double rate = P.snv_rate + P.indel_rate;
    if (rate > 0) {
        uint64_t x = 0;
        for (;;) {
            x += r.geom(1.0 / rate);
            if (x >= L) break;
            if (r.uni() < P.snv_rate / rate) ev.push_back({x, 0, 1});
            else { const uint64_t l = std::min<uint64_t>(r.geom(P.indel_mean), P.indel_max); ev.push_back({x, r.below(2) ? 1 : 2, l}); }
        }
    }
    for (int k = 0; k < n_sv; k++) {
        const uint64_t l = r.range(P.sv_min, P.sv_max);
        if (L < 2 * l + 2) continue;
        ev.push_back({r.below(L - l), r.below(2) ? 1 : 2, l});
    }
    std::sort(ev.begin(), ev.end(), [](const Ev& a, const Ev& b) { return a.pos < b.pos; });
    std::vector<Seg> segs; uint64_t x = 0; std::vector<uint8_t> tmp;
    for (const Ev& e : ev) {
        if (e.pos < x) continue;                              // inside an earlier deletion
        push_copy(segs, (int64_t)(base + x), e.pos - x); x = e.pos;
        if (e.type == 0) {
            const uint8_t rb = R.seq[base + x], u = up(rb);
            uint8_t alt;
            if (u == 'A' || u == 'C' || u == 'G' || u == 'T') {
                const char* B = "ACGT"; const int k = (int)(strchr(B, u) - B);
                alt = (uint8_t)B[(k + 1 + r.below(3)) % 4];
                if (rb != u) alt |= 0x20;                     // case follows the source position
            } else alt = rb;
            push_lit(segs, lit, &alt, 1); x += 1;
        } else if (e.type == 1) {
            tmp.resize(e.len);
            for (auto& t : tmp)                                // inserted sequence: random, upper case
                t = (P.ins_odd > 0 && r.uni() < P.ins_odd) ? (uint8_t)"NNNNRYKMSW"[r.below(10)] : (uint8_t)"ACGT"[r.below(4)];
            push_lit(segs, lit, tmp.data(), e.len);
        } else {
            x = std::min(L, x + e.len);
        }
    }
    push_copy(segs, (int64_t)(base + x), L - x);
    return segs;
}

// cut a segment list at haplotype offsets; reverse-complement a piece
std::vector<Seg> slice(const std::vector<Seg>& s, uint64_t a, uint64_t b) {
    std::vector<Seg> out; uint64_t h = 0;
    for (const Seg& g : s) {
        const uint64_t g0 = h, g1 = h + g.len; h = g1;
        if (g1 <= a || g0 >= b) continue;
        const uint64_t x0 = std::max(a, g0), x1 = std::min(b, g1);
        Seg n = g; n.len = x1 - x0;
        if (g.ref >= 0) n.ref = g.ref + (int64_t)(x0 - g0); else n.lo = g.lo + (x0 - g0);
        out.push_back(n);
    }
    return out;
}
std::vector<Seg> revcomp(const std::vector<Seg>& s, std::vector<uint8_t>& lit) {
    std::vector<Seg> out;
    for (auto it = s.rbegin(); it != s.rend(); ++it) {
        Seg n = *it;
        if (n.ref >= 0) n.dir ^= 1;
        else {
            const uint64_t lo = lit.size();
            for (uint64_t i = 0; i < n.len; i++) lit.push_back(COMP_T[lit[n.lo + n.len - 1 - i]]);
            n.lo = lo;
        }
        out.push_back(n);
    }
    return out;
}

Hap make_hap(const Reference& R, const AsmParams& P, int a) {
    Hap H; Rng r(mix(P.seed, 1000003ull * (uint64_t)a + 17));
    const int nc = (int)R.len.size();
    std::vector<int> svs(nc, P.sv_per_contig);
    if (P.sv_per_asm > 0) {             // SVs spread over contigs by length
        uint64_t tot = 0; for (auto l : R.len) tot += l;
        for (int k = 0; k < P.sv_per_asm; k++) { uint64_t x = r.below(tot); int c = 0; while (x >= R.len[c]) { x -= R.len[c]; c++; } svs[c]++; }
    }
    int rec_no = 0;
    for (int c = 0; c < nc; c++) {
        std::vector<Seg> segs = mutate_contig(R, c, P, r, svs[c], H.lit);
        uint64_t hl = 0; for (auto& g : segs) hl += g.len;
        std::vector<uint64_t> cuts = {0, hl};
        if (P.frag_max > 0 && hl > 1000) {
            const int k = (int)r.range((uint64_t)P.frag_min, (uint64_t)P.frag_max);
            for (int i = 1; i < k; i++) cuts.push_back(r.below(hl));
            std::sort(cuts.begin(), cuts.end()); cuts.erase(std::unique(cuts.begin(), cuts.end()), cuts.end());
        }
        for (size_t i = 0; i + 1 < cuts.size(); i++) {
            Record rc;
            rc.segs = cuts.size() == 2 ? segs : slice(segs, cuts[i], cuts[i + 1]);
            const bool flip = P.rc_piece > 0 && r.uni() < P.rc_piece;
            if (flip) rc.segs = revcomp(rc.segs, H.lit);
            rc.len = cuts[i + 1] - cuts[i];
            rc.hdr = "h" + std::to_string(a) + "_" + R.names[c] + (cuts.size() > 2 ? "_p" + std::to_string(i) : "") + (flip ? " strand=-" : " strand=+");
            rc.lw = (rec_no++ % 2 == 0) ? (uint32_t)P.line_width_a : (uint32_t)P.line_width_b;
            H.rec.push_back(std::move(rc));
        }
    }
    return H;
}

// materialise haplotype stream bytes [h0, h1) (case kept) through a cursor over the concatenated records
struct Cursor {
    const Reference& R; const Hap& H; std::vector<const Seg*> segs; std::vector<uint64_t> start; size_t k = 0;
    Cursor(const Reference& r, const Hap& h) : R(r), H(h) {
        uint64_t x = 0;
        for (auto& rc : H.rec) for (auto& g : rc.segs) { segs.push_back(&g); start.push_back(x); x += g.len; }
        start.push_back(x);
    }
    uint64_t total() const { return start.back(); }
    void seek(uint64_t h) {                 // segment containing h (monotone use is O(1) amortised)
        if (k >= segs.size() || start[k] > h) k = (size_t)(std::upper_bound(start.begin(), start.end(), h) - start.begin()) - 1;
        while (k + 1 < segs.size() && start[k + 1] <= h) k++;
    }
    void fill(uint64_t h0, uint64_t h1, uint8_t* out) {
        seek(h0);
        uint64_t h = h0;
        while (h < h1) {
            const Seg& g = *segs[k]; const uint64_t g0 = start[k], n = std::min(h1, g0 + g.len) - h, off = h - g0;
            if (g.ref < 0) memcpy(out + (h - h0), &H.lit[g.lo + off], n);
            else if (!g.dir) memcpy(out + (h - h0), &R.seq[(uint64_t)g.ref + off], n);
            else { const uint64_t top = (uint64_t)g.ref + g.len - 1 - off; for (uint64_t i = 0; i < n; i++) out[h - h0 + i] = COMP_T[R.seq[top - i]]; }
            h += n; if (h < h1) k++;
        }
    }
};

// ------------------------------------------------------------------ encoder
// A block's coded stream is a list of items in the order the decoder reads them: a symbol of one of the model contexts,
// or up to 16 raw bits (ctx RAW). The list is counted into the model tables first, then rANS-coded back to front.
constexpr uint8_t RAW = 255;
struct Sym { uint8_t ctx; uint8_t s; uint8_t nb; uint8_t pad; uint32_t raw; };
struct Diag {
    int64_t c; uint32_t dir;
    bool operator==(const Diag& o) const { return c == o.c && dir == o.dir; }
};
inline uint64_t zigzag(int64_t d) { return d < 0 ? 2 * (uint64_t)(-(d + 1)) + 1 : 2 * (uint64_t)d; }

// the largest value the bucket code holds: the top symbol of a big alphabet with all its extra bits set
constexpr uint64_t BUCKET_MAX = pvc::unbucket(pvc::BIG_ALPHA - 1, (1ull << pvc::nbits_of(pvc::BIG_ALPHA - 1)) - 1);

struct Event { uint32_t at, L; uint32_t dir; uint64_t p; };   // reference copy at block offset `at`

// The four most recent copy diagonals, most recent first: a diagonal used again moves to the front, a new one is put
// there and pushes the oldest out (the decoder keeps the same list; it is what K_REP and K_FLIP index).
struct DiagCache {
    Diag d[4]; int n = 0;
    void reset(const Diag& g) { d[0] = g; n = 1; }
    void touch(const Diag& g) {
        int j = (int)(std::find(d, d + n, g) - d);
        if (j == n) j = n < 4 ? n++ : 3;
        std::rotate(d, d + j, d + j + 1);
        d[0] = g;
    }
};

// Turns one block's literal runs and copy events into coded items.
class BlockCoder {
  public:
    BlockCoder(const uint8_t* ref, uint64_t ref_n, std::vector<Sym>& out) : ref_(ref), ref_n_(ref_n), out_(out) {}

    void encode(const uint8_t* blk, uint32_t blen, const std::vector<Event>& ev, Diag start) {
        cache_.reset(start);
        last_kind_ = -1;
        uint32_t o = 0;
        for (size_t e = 0; o < blen; e++) {
            const uint32_t at = e < ev.size() ? ev[e].at : blen;
            const uint32_t run = at - o;
            literal_run(blk + o, o, run);
            o = at;
            if (o == blen) break;
            copy(ev[e], o, run);
            o += ev[e].L;
        }
    }

  private:
    void symbol(int ctx, uint32_t s) { out_.push_back({(uint8_t)ctx, (uint8_t)s, 0, 0, 0}); }
    void bits(uint64_t v, uint32_t nb) {          // raw bits, 16 at most per item, the low part first
        for (uint32_t sh = 0; sh < nb; sh += 16) {
            const uint32_t k = std::min(16u, nb - sh);
            out_.push_back({RAW, 0, (uint8_t)k, 0, (uint32_t)((v >> sh) & ((1u << k) - 1))});
        }
    }
    // v in the bucket code: 0..15 are their own symbols; above, the symbol names the top bit and the two bits under
    // it, and the bits below those follow raw
    void value(int ctx, uint64_t v) {
        if (v < 16) { symbol(ctx, (uint32_t)v); return; }
        const uint32_t top = 63 - (uint32_t)__builtin_clzll(v), low = top - 2;
        const uint32_t s = 4 * top - 4 + (uint32_t)(v >> low);          // v >> low is 4..7: the top bit and two more
        symbol(ctx, s);
        bits(v & ((1ull << low) - 1), pvc::nbits_of(s));
    }
    uint32_t ref_base(uint32_t o) const {          // base code of the reference along the current diagonal at offset o
        const int64_t q = pvc::diag_locus(cache_.d[0].c, cache_.d[0].dir, o);
        if (q < 0 || (uint64_t)q >= ref_n_) return 4;
        const uint8_t x = up(ref_[q]);
        return (uint32_t)pvc::base4(cache_.d[0].dir ? pvc::comp(x) : x);
    }
    static uint32_t code_of(uint8_t b) {           // A C G T N, 5 = any other byte (escaped: 8 raw bits follow)
        switch (b) { case 'A': return 0; case 'C': return 1; case 'G': return 2; case 'T': return 3; case 'N': return 4; default: return 5; }
    }
    void literal_run(const uint8_t* lit, uint32_t o, uint32_t run) {
        value(pvc::C_LL + pvc::kclass(last_kind_), run);
        // short runs: context = the reference base the diagonal predicts, and whether this is the run's first literal;
        // long runs: order 2 over the run's own previous two literals (N and escapes count as A)
        uint32_t hist = 0, h1 = 0, h2 = 0;
        for (uint32_t j = 0; j < run; j++) {
            const uint32_t s = code_of(lit[j]);
            const int ctx = run <= 8 ? pvc::C_LITR + (int)(2 * ref_base(o + j) + (j == 0))
                                     : pvc::C_LIT2 + (hist == 0 ? 16 : hist == 1 ? (int)h1 : (int)(4 * h2 + h1));
            symbol(ctx, s);
            if (s == 5) bits(lit[j], 8);
            h2 = h1; h1 = s < 4 ? s : 0; hist += hist < 2;
        }
    }
    // The cheapest way to name the event's position from the cached diagonals, by the extra raw bits its value costs
    // plus 3 bits per coded symbol: the same diagonal (CONT, free), the front diagonal moved (DELTA), another cached
    // one moved (REP), one of the other strand (FLIP), or the absolute position (ABS: strand + 32 raw bits).
    struct Choice { int kind, k; uint64_t z; uint32_t cost; };
    static uint32_t extra_bits(uint64_t z) { return z < 16 ? 0u : 61u - (uint32_t)__builtin_clzll(z); }
    Choice choose(const Event& v, uint32_t o) const {
        Choice best{pvc::K_ABS, 0, 0, 3 + 32};
        for (int k = 0; k < cache_.n; k++) {
            const Diag& g = cache_.d[k];
            const bool same = g.dir == v.dir;
            const int64_t want = same ? pvc::diag_expect(g.c, g.dir, o, v.L) : pvc::diag_locus(g.c, g.dir, o);
            const uint64_t z = zigzag((int64_t)v.p - want);
            if (z > BUCKET_MAX) continue;
            Choice c;
            if (!same) c = {pvc::K_FLIP, k, z, 6 + extra_bits(z)};
            else if (k == 0) c = z == 0 ? Choice{pvc::K_CONT, 0, 0, 0} : Choice{pvc::K_DELTA, 0, z, 3 + extra_bits(z)};
            else c = {pvc::K_REP, k, z, 6 + extra_bits(z)};
            if (c.cost < best.cost) best = c;
        }
        return best;
    }
    void copy(const Event& v, uint32_t o, uint32_t run) {
        const Choice c = choose(v, o);
        symbol(pvc::C_KIND + pvc::llc(run) * 4 + pvc::kclass(last_kind_), (uint32_t)c.kind);
        switch (c.kind) {
            case pvc::K_DELTA: value(pvc::C_DELTA + (run ? 1 : 0), c.z); break;
            case pvc::K_REP: symbol(pvc::C_REPK, (uint32_t)(c.k - 1)); value(pvc::C_REPD, c.z); break;
            case pvc::K_FLIP: symbol(pvc::C_FLIPK, (uint32_t)c.k); value(pvc::C_FLIPD, c.z); break;
            case pvc::K_ABS: symbol(pvc::C_DIR, v.dir); bits(v.p, 32); break;
            default: break;                                               // K_CONT: nothing more
        }
        value(pvc::C_LEN + c.kind, v.L - pvc::MIN_LEN);
        cache_.touch({pvc::diag_of(v.dir, v.p, o, v.L), v.dir});
        last_kind_ = c.kind;
    }

    const uint8_t* ref_; uint64_t ref_n_; std::vector<Sym>& out_;
    DiagCache cache_; int last_kind_ = -1;
};

// A context's frequencies from its symbol counts: every symbol seen gets 1, and the rest of the 4096 is apportioned by
// largest remainders (Hamilton's method) - each seen symbol its whole quota of the rest, cnt x rest / total, and the
// units still left one each to the largest fractional parts, lowest symbol first on ties. Exact integer arithmetic.
void normalise(const uint64_t* cnt, int n, uint16_t* f) {
    std::fill(f, f + n, (uint16_t)0);
    uint64_t total = 0;
    int seen = 0;
    for (int s = 0; s < n; s++) { total += cnt[s]; seen += cnt[s] != 0; }
    if (!total) return;
    const uint64_t rest = pvc::M - (uint64_t)seen;
    std::vector<std::pair<uint64_t, int>> frac;                 // (remainder of cnt x rest / total, symbol)
    uint64_t given = 0;
    for (int s = 0; s < n; s++) {
        if (!cnt[s]) continue;
        const unsigned __int128 share = (unsigned __int128)cnt[s] * rest;
        const uint64_t whole = (uint64_t)(share / total);
        f[s] = (uint16_t)(1 + whole);
        given += whole;
        frac.emplace_back((uint64_t)(share % total), s);
    }
    std::stable_sort(frac.begin(), frac.end(), [](const auto& a, const auto& b) { return a.first > b.first; });
    for (uint64_t k = 0; k < rest - given; k++) f[frac[k].second]++;
}

// rANS coder of one block. The decoder starts from a 24-bit state (3 bytes, low first) and reads further bytes as its
// renormalisation needs them, so the coder runs over the items back to front and sheds the state's low bytes before a
// step that would push it past 2^24; the bytes come out in the reverse of the order the decoder reads them and are
// turned around once at the end.
class RansWriter {
  public:
    RansWriter(const uint16_t* freq, const uint16_t* cum) : freq_(freq), cum_(cum) {}
    void block(const Sym* first, const Sym* last, std::vector<uint8_t>& payload) {
        x_ = pvc::RANS_L;
        back_.clear();
        for (const Sym* it = last; it != first;) {
            const Sym& s = *--it;
            if (s.ctx == RAW) {
                shed(1u << (24 - s.nb));
                x_ = (x_ << s.nb) | s.raw;
            } else {
                const size_t at = (size_t)s.ctx * pvc::BIG_ALPHA + s.s;
                const uint32_t f = freq_[at];
                shed(f << (24 - pvc::PROB_BITS));
                x_ = (x_ / f) * pvc::M + x_ % f + cum_[at];
            }
        }
        for (int k = 2; k >= 0; k--) back_.push_back((uint8_t)(x_ >> (8 * k)));   // read first: low, middle, high
        payload.insert(payload.end(), back_.rbegin(), back_.rend());
    }

  private:
    void shed(uint32_t bound) { for (; x_ >= bound; x_ >>= 8) back_.push_back((uint8_t)x_); }
    const uint16_t* freq_; const uint16_t* cum_;
    uint32_t x_ = pvc::RANS_L;
    std::vector<uint8_t> back_;
};

void leb(std::vector<uint8_t>& o, uint64_t v) { while (v >= 0x80) { o.push_back((uint8_t)(v | 0x80)); v >>= 7; } o.push_back((uint8_t)v); }
template <class T> void put(std::vector<uint8_t>& o, T v) { o.insert(o.end(), (uint8_t*)&v, (uint8_t*)&v + sizeof v); }

struct Stats { std::atomic<uint64_t> bases{0}, blocks{0}, payload{0}, files{0}, file_bytes{0}; };

// encode haplotype `a` to <dir>/<prefix><a>.<Q/1024>k.rr3
bool encode_asm(const Reference& R, const uint8_t ref_sha[32], const std::string& ref_name, const AsmParams& P, int a, const std::string& dir, Stats& S, std::string& err) {
    double t0 = now_s();
    Hap H = make_hap(R, P, a);
    Cursor cur(R, H);
    phase("haplotype segments", t0); t0 = now_s();
    const uint64_t n = cur.total(), Q = (uint64_t)P.Q, nb = (n + Q - 1) / Q;
    const uint8_t* ref = R.seq.data(); const uint64_t ref_n = R.seq.size();
    // upper-case reference for literal contexts
    // pass A: stream bytes -> base XXH3, FASTA XXH3, block XXH3 (upper case), lower-case runs
    pvx::Stream hb, hf; std::vector<uint64_t> bh; if (P.block_hashes) bh.resize(nb);
    std::vector<uint8_t> runs; uint64_t nruns = 0, last_end = 0; bool in_low = false; uint64_t low_start = 0;
    {
        const uint64_t CH = Q * 256; std::vector<uint8_t> buf(CH), upb(Q), fa(CH + CH / 8 + 4096);
        size_t ri = 0; uint64_t rpos = 0;   // record index, offset within record
        size_t fw = 0;                      // FASTA text pending in fa
        auto fasta_header = [&](size_t r) {
            const std::string h = ">" + H.rec[r].hdr + "\n";
            if (fw + h.size() > fa.size()) { hf.update(fa.data(), fw); fw = 0; }
            if (h.size() > fa.size()) hf.update(h.data(), h.size()); else { memcpy(&fa[fw], h.data(), h.size()); fw += h.size(); }
        };
        if (!H.rec.empty()) fasta_header(0);
        for (uint64_t h0 = 0; h0 < n; h0 += CH) {
            const uint64_t h1 = std::min(n, h0 + CH);
            cur.fill(h0, h1, buf.data());
            hb.update(buf.data(), h1 - h0);
            if (R.has_lower)
                for (uint64_t x = h0; x < h1; x++) {             // case runs
                    const bool low = buf[x - h0] >= 'a' && buf[x - h0] <= 'z';
                    if (low && !in_low) { in_low = true; low_start = x; }
                    else if (!low && in_low) { in_low = false; leb(runs, low_start - last_end); leb(runs, x - low_start); last_end = x; nruns++; }
                }
            if (P.block_hashes)
                for (uint64_t b = h0 / Q; b * Q < h1; b++) {
                    const uint64_t bl = std::min(Q, n - b * Q);
                    for (uint64_t i = 0; i < bl; i++) upb[i] = up(buf[b * Q - h0 + i]);
                    bh[b] = pvx::xxh3_64(upb.data(), bl);
                }
            // FASTA text: lines of the record's width, a header at each record start
            uint64_t x = h0;
            while (x < h1) {
                while (ri < H.rec.size() && rpos == H.rec[ri].len) { ri++; rpos = 0; if (ri < H.rec.size()) fasta_header(ri); }
                const Record& rc = H.rec[ri];
                const uint64_t line_left = rc.lw - (rpos % rc.lw), k = std::min({line_left, rc.len - rpos, h1 - x});
                if (fw + k + 1 > fa.size()) { hf.update(fa.data(), fw); fw = 0; }
                memcpy(&fa[fw], &buf[x - h0], k); fw += k; x += k; rpos += k;
                if (rpos % rc.lw == 0 || rpos == rc.len) fa[fw++] = '\n';
            }
        }
        while (ri < H.rec.size() && rpos == H.rec[ri].len) { ri++; rpos = 0; if (ri < H.rec.size()) fasta_header(ri); }
        hf.update(fa.data(), fw);
        if (in_low) { leb(runs, low_start - last_end); leb(runs, n - low_start); nruns++; }
    }
    phase("pass A (hashes)", t0); t0 = now_s();
    // pass B: per block events -> symbols; model counts
    std::vector<Sym> sy; std::vector<uint64_t> sy_off(nb + 1, 0); std::vector<Diag> st(nb);
    std::vector<uint64_t> cnt((size_t)pvc::NCTX * pvc::BIG_ALPHA, 0);
    {
        std::vector<uint8_t> blk(Q); std::vector<Event> ev;
        BlockCoder coder(ref, ref_n, sy);
        // the diagonal of a copy segment g (starting at stream position g0) relative to a block starting at b0:
        // forward c = ref + (b0 - g0) (locus c + o); reverse complement c = top + g0 - b0 (locus c - o)
        auto diag_at = [](const Seg& g, uint64_t g0, uint64_t b0) -> Diag {
            return g.dir ? Diag{g.ref + (int64_t)g.len - 1 + (int64_t)g0 - (int64_t)b0, 1u} : Diag{g.ref + (int64_t)b0 - (int64_t)g0, 0u};
        };
        for (uint64_t b = 0; b < nb; b++) {
            const uint64_t b0 = b * Q, blen = std::min(Q, n - b0);
            // start diagonal: the copy segment covering the block start, else the last copy segment before it
            cur.seek(b0);
            {
                size_t k = cur.k;
                while (k > 0 && cur.segs[k]->ref < 0) k--;
                st[b] = cur.segs[k]->ref >= 0 ? diag_at(*cur.segs[k], cur.start[k], b0) : Diag{0, 0};
            }
            ev.clear();
            uint64_t h = b0;
            while (h < b0 + blen) {
                cur.seek(h);
                const Seg& g = *cur.segs[cur.k]; const uint64_t g0 = cur.start[cur.k], e = std::min(b0 + blen, g0 + g.len), off = h - g0;
                if (g.ref >= 0 && e - h >= pvc::MIN_LEN) {     // shorter copy pieces stay literals
                    const uint64_t L = e - h;
                    const uint64_t p = g.dir ? (uint64_t)g.ref + g.len - off - L : (uint64_t)g.ref + off;
                    ev.push_back({(uint32_t)(h - b0), (uint32_t)L, g.dir, p});
                }
                h = e;
            }
            // literal bytes: only the gaps between copy events are read by the symbol coder
            {
                uint32_t o = 0;
                for (size_t k = 0; k <= ev.size(); k++) {
                    const uint32_t nx = k < ev.size() ? ev[k].at : (uint32_t)blen;
                    if (nx > o) { cur.fill(b0 + o, b0 + nx, &blk[o]); for (uint32_t i = o; i < nx; i++) blk[i] = up(blk[i]); }
                    if (k < ev.size()) o = ev[k].at + ev[k].L;
                }
            }
            const size_t s0 = sy.size();
            coder.encode(blk.data(), (uint32_t)blen, ev, st[b]);
            for (size_t k = s0; k < sy.size(); k++) if (sy[k].ctx != RAW) cnt[(size_t)sy[k].ctx * pvc::BIG_ALPHA + sy[k].s]++;
            sy_off[b + 1] = sy.size();
        }
    }
    phase("pass B (symbols)", t0); t0 = now_s();
    // tables
    std::vector<uint16_t> freq((size_t)pvc::NCTX * pvc::BIG_ALPHA, 0), cum((size_t)pvc::NCTX * pvc::BIG_ALPHA, 0);
    for (int c = 0; c < pvc::NCTX; c++) {
        normalise(&cnt[(size_t)c * pvc::BIG_ALPHA], pvc::alpha_of(c), &freq[(size_t)c * pvc::BIG_ALPHA]);
        uint32_t acc = 0; for (int s = 0; s < pvc::BIG_ALPHA; s++) { cum[(size_t)c * pvc::BIG_ALPHA + s] = (uint16_t)acc; acc += freq[(size_t)c * pvc::BIG_ALPHA + s]; }
    }
    // pass C: rANS per block
    std::vector<uint8_t> pay; std::vector<uint64_t> plen(nb);
    RansWriter rans(freq.data(), cum.data());
    for (uint64_t b = 0; b < nb; b++) {
        const size_t before = pay.size();
        rans.block(sy.data() + sy_off[b], sy.data() + sy_off[b + 1], pay);
        plen[b] = pay.size() - before;
    }
    std::vector<Sym>().swap(sy);
    phase("pass C (rANS)", t0); t0 = now_s();
    if (pay.size() >= (1ull << 32)) { err = "payload over 4 GiB"; return false; }
    // meta
    std::vector<uint8_t> M;
    put<uint32_t>(M, (uint32_t)H.rec.size());
    for (auto& rc : H.rec) { put<uint32_t>(M, (uint32_t)rc.hdr.size()); M.insert(M.end(), rc.hdr.begin(), rc.hdr.end()); put<uint64_t>(M, rc.len); put<uint32_t>(M, rc.lw); }
    put<uint64_t>(M, nruns); M.insert(M.end(), runs.begin(), runs.end());
    for (int c = 0; c < pvc::NCTX; c++) for (int s = 0; s < pvc::alpha_of(c); s++) leb(M, freq[(size_t)c * pvc::BIG_ALPHA + s]);
    int64_t prevc = 0; uint32_t prevd = 0;
    for (uint64_t b = 0; b < nb; b++) {
        leb(M, plen[b]);
        const int64_t pred = b == 0 ? 0 : (prevd ? prevc - (int64_t)Q : prevc + (int64_t)Q);
        leb(M, zigzag(st[b].c - pred) * 2 + st[b].dir);
        prevc = st[b].c; prevd = st[b].dir;
    }
    std::vector<uint8_t> MZ(ZSTD_compressBound(M.size()));
    const size_t mz = ZSTD_compress(MZ.data(), MZ.size(), M.data(), M.size(), P.zstd_level);
    if (ZSTD_isError(mz)) { err = "zstd"; return false; }
    MZ.resize(mz);
    // header
    std::vector<uint8_t> o(136, 0);
    memcpy(&o[0], "RFRL3V1\0", 8);
    auto p32 = [&](size_t at, uint32_t v) { memcpy(&o[at], &v, 4); };
    auto p64 = [&](size_t at, uint64_t v) { memcpy(&o[at], &v, 8); };
    p32(8, 1); p32(12, (uint32_t)Q); p32(16, P.block_hashes ? 1 : 0); p32(20, 0);
    memcpy(&o[24], ref_sha, 32); p64(56, ref_n); p64(64, n); p64(72, nb); p64(80, hf.digest()); p64(88, hb.digest());
    p64(96, MZ.size()); p64(104, M.size()); p64(112, bh.size() * 8); p64(120, pay.size());
    const uint16_t nl = (uint16_t)std::min<size_t>(ref_name.size(), 65535);
    o.push_back((uint8_t)nl); o.push_back((uint8_t)(nl >> 8)); o.insert(o.end(), ref_name.begin(), ref_name.begin() + nl);
    o.insert(o.end(), MZ.begin(), MZ.end());
    if (!bh.empty()) o.insert(o.end(), (uint8_t*)bh.data(), (uint8_t*)bh.data() + bh.size() * 8);
    p64(128, pvx::xxh3_64(o.data(), o.size()));
    char name[512]; snprintf(name, sizeof name, "%s/%s%03d.q%uk.rr3", dir.c_str(), P.prefix, a, (unsigned)(Q / 1024));
    FILE* f = fopen(name, "wb"); if (!f) { err = std::string("cannot write ") + name; return false; }
    fwrite(o.data(), 1, o.size(), f); fwrite(pay.data(), 1, pay.size(), f);
    if (fclose(f)) { err = std::string("short write ") + name; return false; }
    phase("meta + write", t0);
    S.bases += n; S.blocks += nb; S.payload += pay.size(); S.files++; S.file_bytes += o.size() + pay.size();
    return true;
}

// SHA-256 of the upper-cased reference, streamed in chunks; the system libcrypto when present (SHA-NI / AVX2),
// else the portable implementation
void sha256_upper(const std::vector<uint8_t>& seq, uint8_t out[32]) {
    struct Ctx { uint8_t opaque[256]; };
    typedef int (*Init)(void*); typedef int (*Upd)(void*, const void*, size_t); typedef int (*Fin)(unsigned char*, void*);
    void* h = dlopen("libcrypto.so.3", RTLD_NOW | RTLD_LOCAL);
    Init fi = h ? (Init)dlsym(h, "SHA256_Init") : nullptr; Upd fu = h ? (Upd)dlsym(h, "SHA256_Update") : nullptr; Fin ff = h ? (Fin)dlsym(h, "SHA256_Final") : nullptr;
    std::vector<uint8_t> chunk(1 << 20);
    Ctx ctx; pvs::Sha256 portable; const bool lib = fi && fu && ff;
    if (lib) fi(&ctx);
    for (size_t i = 0; i < seq.size(); i += chunk.size()) {
        const size_t k = std::min(chunk.size(), seq.size() - i);
        for (size_t j = 0; j < k; j++) chunk[j] = up(seq[i + j]);
        if (lib) fu(&ctx, chunk.data(), k); else portable.update(chunk.data(), k);
    }
    if (lib) ff(out, &ctx); else portable.digest(out);
}

}  // namespace

extern "C" {

// Make <dir>/reference.fa and n_asm archives. Returns 0, or 1 with a message in err. stats (may be NULL): bases,
// blocks, payload bytes, files, file bytes, reference bases.
int cg_make_cohort(const char* dir, const RefParams* RP, const AsmParams* AP, uint64_t* stats, char* err, size_t errcap) {
    std::string e;
    try {
        const int T = std::max(1, AP->threads);
        double t0 = now_s();
        Reference R; make_reference(*RP, R, T);
        phase("reference bases", t0); t0 = now_s();
        const std::string rpath = std::string(dir) + "/reference.fa";
        if (!write_fasta_ref(R, RP->line_width, rpath)) { snprintf(err, errcap, "cannot write %s", rpath.c_str()); return 1; }
        phase("reference FASTA write", t0); t0 = now_s();
        uint8_t sha[32];
        sha256_upper(R.seq, sha);
        phase("reference SHA-256", t0);
        t0 = now_s();
        Stats S; std::mutex mu; std::atomic<int> next{0}, finished{0}; std::vector<std::thread> th;
        for (int t = 0; t < std::min(T, AP->n_asm); t++) th.emplace_back([&] {
            for (;;) {
                const int a = next.fetch_add(1); if (a >= AP->n_asm) break;
                std::string m;
                if (!encode_asm(R, sha, "reference.fa", *AP, a, dir, S, m)) { std::lock_guard<std::mutex> g(mu); if (e.empty()) e = m; }
                // progress for long cohorts (a caller that waits minutes sees it moving)
                const int done = ++finished;
                if (AP->n_asm >= 64 && (done % 32 == 0 || done == AP->n_asm)) {
                    fprintf(stderr, "cohortgen: %d / %d haplotypes encoded, %.0f s\n", done, AP->n_asm, now_s() - t0);
                    // and to a file named by COHORTGEN_PROGRESS, for callers whose stderr is captured
                    if (const char* pf = getenv("COHORTGEN_PROGRESS")) {
                        std::lock_guard<std::mutex> g(mu);
                        if (FILE* f = fopen(pf, "a")) { fprintf(f, "cohortgen: %d / %d haplotypes encoded, %.0f s\n", done, AP->n_asm, now_s() - t0); fclose(f); }
                    }
                }
            }
        });
        for (auto& x : th) x.join();
        if (!e.empty()) { snprintf(err, errcap, "%s", e.c_str()); return 1; }
        if (stats) { stats[0] = S.bases; stats[1] = S.blocks; stats[2] = S.payload; stats[3] = S.files; stats[4] = S.file_bytes; stats[5] = R.seq.size(); }
        return 0;
    } catch (const std::exception& x) { snprintf(err, errcap, "%s", x.what()); return 1; }
}

}  // extern "C"
