// pv_host.cpp - host side of the MI355X refrel3 v1 decode path: the decoded reference, archives opened with every
// check of the format before any decode, their arrays pooled for one device copy, the GPU model tables, contig
// tables, and the FASTA layout / XXH3 of a decoded stream. Exposed through the C ABI of include/panvram_amd.h.
//
// Behaviour follows the reference host core: reference loading (csrc/pv_v1.h:42-53 fasta_bases_inplace,
// csrc/pv_core.cpp:35-41), open with checks in the order of csrc/pv_v1.h:99-146 (open_v1), pooling
// (csrc/pv_core.cpp:65-90), FASTA rebuild / XXH3 (csrc/pv_core.cpp:138-176). Error messages keep the reference's
// wording ("<path>: refused: <why>") because callers match on them.
#include "../../include/panvram_amd.h"
#include "pv_codec.h"
#include "pv_sha256.h"
#include "pv_xxh3.h"

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <new>
#include <vector>

// zstd (system libzstd.so.1; only the frame queries and the one-shot decompressor are used, for the meta section)
extern "C" {
unsigned long long ZSTD_getFrameContentSize(const void* src, size_t srcSize);
size_t ZSTD_findFrameCompressedSize(const void* src, size_t srcSize);
size_t ZSTD_decompress(void* dst, size_t dstCapacity, const void* src, size_t compressedSize);
}

namespace {

struct FormatErr : std::runtime_error { using std::runtime_error::runtime_error; };
struct ArgErr : std::runtime_error { using std::runtime_error::runtime_error; };

constexpr uint32_t HDR = 136, VERSION = 1, F_BLOCKHASH = 1;
constexpr char MAGIC[8] = {'R', 'F', 'R', 'L', '3', 'V', '1', 0};

inline uint64_t rd64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }
inline uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
inline bool block_size_ok(uint32_t q) { return q == 1024 || q == 2048 || q == 4096 || q == 16384; }
std::string hex(const uint8_t* p, size_t n) {
    static const char* d = "0123456789abcdef"; std::string s;
    for (size_t i = 0; i < n; i++) { s += d[p[i] >> 4]; s += d[p[i] & 15]; }
    return s;
}

std::vector<uint8_t> read_file(const std::string& p) {
    FILE* f = fopen(p.c_str(), "rb");
    if (!f) throw FormatErr(p + ": cannot open");
    fseek(f, 0, SEEK_END); const long s = ftell(f); fseek(f, 0, SEEK_SET);
    std::vector<uint8_t> v((size_t)std::max<long>(s, 0));
    const size_t r = v.empty() ? 0 : fread(v.data(), 1, v.size(), f); fclose(f);
    if (r != v.size()) throw FormatErr(p + ": short read");
    return v;
}

// A FASTA file's bytes -> its bases, in place: header lines and line ends dropped, a..z upper-cased
// (reference csrc/pv_v1.h:42-53). Returns the base count.
uint64_t fasta_to_bases(uint8_t* b, uint64_t n, const std::string& path) {
    if (!n || b[0] != '>') throw FormatErr(path + ": not FASTA (no header at byte 0)");
    uint64_t i = 0, w = 0;
    while (i < n) {
        const uint8_t* e = (const uint8_t*)memchr(b + i, '\n', n - i);
        if (b[i] == '>') {
            if (!e) throw FormatErr(path + ": header without line end");
            i = (uint64_t)(e - b) + 1; continue;
        }
        if (!e) throw FormatErr(path + ": no final line end");
        const uint64_t le = (uint64_t)(e - b);
        for (uint64_t k = i; k < le; k++) { const uint8_t c = b[k]; b[w++] = (c >= 'a' && c <= 'z') ? (uint8_t)(c - 32) : c; }
        i = le + 1;
    }
    return w;
}

template <class F> void parallel_for(uint64_t n, int threads, F&& f) {
    if (!n) return;
    const int T = (int)std::max<uint64_t>(1, std::min<uint64_t>((uint64_t)std::max(1, threads), n));
    std::atomic<uint64_t> next{0}; std::vector<std::thread> th;
    for (int t = 0; t < T; t++) th.emplace_back([&] { for (;;) { const uint64_t i = next.fetch_add(1); if (i >= n) break; f(i); } });
    for (auto& x : th) x.join();
}
int host_threads() { const unsigned h = std::thread::hardware_concurrency(); return h ? (int)h : 4; }

struct Contig { std::string hdr, name; uint64_t len = 0, boff = 0; uint32_t lw = 0; };

struct Archive {
    std::string path, refname;
    uint32_t Q = 0, flags = 0;
    uint64_t nbases = 0, nb = 0, fasta_xxh = 0, bases_xxh = 0, file_bytes = 0, payload_bytes = 0;
    std::vector<Contig> rec;
    std::vector<int64_t> low_s, low_l;
    std::vector<uint64_t> hashes;
    std::vector<uint16_t> freq;        // [61][104]
    std::vector<uint32_t> off;         // nb + 1
    std::vector<int64_t> st;           // nb + 1 (last = 0)
    std::vector<uint8_t> payload;
};

// Open one archive: every check before any decode, in the reference's order (csrc/pv_v1.h:99-146).
void open_archive(const std::vector<uint8_t>& file, const std::string& path, const uint8_t ref_sha[32], uint64_t ref_n, Archive& X) {
    const uint8_t* a = file.data(); const uint64_t n = file.size();
    auto refuse = [&](const char* why) { throw FormatErr(path + ": refused: " + why); };
    if (n < HDR + 2) refuse("short file");
    if (memcmp(a, MAGIC, 8)) refuse("magic (not refrel3 v1)");
    if (rd32(a + 8) != VERSION) refuse("version");
    X.Q = rd32(a + 12); if (!block_size_ok(X.Q)) refuse("block size");
    X.flags = rd32(a + 16); if (X.flags & ~F_BLOCKHASH) refuse("unknown flags");
    if (rd32(a + 20)) refuse("reserved");
    X.nbases = rd64(a + 64); X.nb = rd64(a + 72); X.fasta_xxh = rd64(a + 80); X.bases_xxh = rd64(a + 88);
    const uint64_t mz = rd64(a + 96), mr = rd64(a + 104), hs = rd64(a + 112), pl = rd64(a + 120);
    const uint16_t nl = (uint16_t)(a[136] | a[137] << 8);
    const uint64_t pstart = (uint64_t)HDR + 2 + nl + mz + hs;
    if (mz > n || hs > n || pl > n || pstart > n || pstart + pl != n) refuse("section sizes");
    if (X.nb != (X.nbases + X.Q - 1) / X.Q || (X.nbases && !X.nb)) refuse("block count");
    if (hs != ((X.flags & F_BLOCKHASH) ? X.nb * 8 : 0)) refuse("hash section size");
    {   // header XXH3 over [0, payload start) with its own field taken as 0
        pvx::Stream h; uint8_t z[8] = {0};
        h.update(a, 128); h.update(z, 8); h.update(a + 136, pstart - 136);
        if (h.digest() != rd64(a + 128)) refuse("header XXH3");
    }
    if (memcmp(a + 24, ref_sha, 32) || rd64(a + 56) != ref_n) refuse("reference SHA-256 / size differs (wrong reference)");
    X.refname.assign((const char*)a + 138, nl);
    const uint8_t* mzp = a + HDR + 2 + nl;
    if (mr > (1ull << 32) || ZSTD_getFrameContentSize(mzp, mz) != mr) refuse("meta frame");
    if (ZSTD_findFrameCompressedSize(mzp, mz) != mz) refuse("meta frame count (exactly one zstd frame)");
    std::vector<uint8_t> M(mr);
    if (ZSTD_decompress(M.data(), mr, mzp, mz) != mr) refuse("meta decompress");

    uint64_t i = 0; bool bad = false;
    auto need = [&](uint64_t k) { if (i + k > M.size()) { bad = true; return false; } return true; };
    auto g64 = [&]() -> uint64_t { if (!need(8)) return 0; const uint64_t v = rd64(&M[i]); i += 8; return v; };
    auto g32 = [&]() -> uint32_t { if (!need(4)) return 0; const uint32_t v = rd32(&M[i]); i += 4; return v; };
    auto leb = [&]() -> uint64_t {
        uint64_t v = 0; int sh = 0;
        for (;;) {
            if (!need(1) || sh > 63) { bad = true; return 0; }
            const uint8_t c = M[i++]; v |= (uint64_t)(c & 0x7F) << sh;
            if (!(c & 0x80)) return v;
            sh += 7;
        }
    };
    // contig table
    const uint32_t nr = g32(); uint64_t bo = 0;
    if (nr > M.size()) refuse("records");
    for (uint32_t r = 0; r < nr && !bad; r++) {
        Contig q; const uint32_t hl = g32(); if (!need(hl)) break;
        q.hdr.assign((const char*)&M[i], hl); i += hl; q.len = g64(); q.lw = g32();
        if (!q.lw && q.len) bad = true;
        q.name = q.hdr.substr(0, q.hdr.find_first_of(" \t")); q.boff = bo; bo += q.len; X.rec.push_back(std::move(q));
    }
    if (bad || bo != X.nbases) refuse("contig table");
    // lower-case runs: LEB128 gap from the previous run's end, LEB128 length
    const uint64_t nlw = g64(); uint64_t last = 0;
    if (nlw > X.nbases) refuse("case runs");
    X.low_s.reserve(nlw); X.low_l.reserve(nlw);
    for (uint64_t k = 0; k < nlw && !bad; k++) {
        const uint64_t g = leb(), l = leb();
        if (last + g + l > X.nbases) { bad = true; break; }
        X.low_s.push_back((int64_t)(last + g)); X.low_l.push_back((int64_t)l); last += g + l;
    }
    if (bad) refuse("case runs");
    // model tables: every context sums to 4096 or is all zero
    X.freq.assign((size_t)pvc::NCTX * pvc::BIG_ALPHA, 0);
    for (int c = 0; c < pvc::NCTX && !bad; c++) {
        uint64_t sum = 0;
        for (int s = 0; s < pvc::alpha_of(c); s++) {
            const uint64_t f = leb(); if (f > pvc::M) bad = true;
            X.freq[(size_t)c * pvc::BIG_ALPHA + s] = (uint16_t)f; sum += f;
        }
        if (sum && sum != pvc::M) bad = true;
    }
    if (bad) refuse("model tables");
    if (pl >= (1ull << 32)) refuse("payload over 4 GiB (pooled offsets are 32-bit)");
    // block table: LEB128 payload length; LEB128 zigzag(c - predicted) * 2 + strand, predicted = previous c +- Q
    X.off.assign(X.nb + 1, 0); X.st.assign(X.nb + 1, 0);
    int64_t prevc = 0; uint32_t prevd = 0; uint32_t acc = 0;
    for (uint64_t b = 0; b < X.nb && !bad; b++) {
        const uint64_t len = leb(); if (len > pl - acc) { bad = true; break; }
        acc += (uint32_t)len; X.off[b + 1] = acc;
        const uint64_t v = leb();
        const int64_t pred = b == 0 ? 0 : (prevd ? prevc - (int64_t)X.Q : prevc + (int64_t)X.Q);
        const int64_t c = (int64_t)((uint64_t)pred + (uint64_t)pvc::unzigzag(v >> 1));
        const uint32_t dir = (uint32_t)(v & 1);
        X.st[b] = (int64_t)(((uint64_t)c << 1) | dir); prevc = c; prevd = dir;
    }
    if (bad || i != M.size() || acc != pl) refuse("block table");
    if (X.flags & F_BLOCKHASH) { X.hashes.resize(X.nb); memcpy(X.hashes.data(), a + HDR + 2 + nl + mz, X.nb * 8); }
    X.payload.assign(a + pstart, a + n); X.payload_bytes = pl; X.file_bytes = n; X.path = path;
}

// GPU model table of one archive (layout in pv_codec.h)
void build_gtab(const Archive& X, uint8_t* out) {
    uint16_t* t = (uint16_t*)out; memset(out, 0, pvc::GTAB_BYTES);
    for (int c = 0; c < pvc::NCTX; c++) {
        const int A = pvc::alpha_of(c), width = A == pvc::BIG_ALPHA ? pvc::BIG_ROW : pvc::SMALL_ROW;
        uint16_t* row = t + pvc::row_of(c); uint32_t cum = 0;
        for (int s = 0; s <= A; s++) { row[s] = (uint16_t)cum; if (s < A) cum += X.freq[(size_t)c * pvc::BIG_ALPHA + s]; }
        for (int s = A + 1; s < width; s++) row[s] = (uint16_t)cum;
    }
    // bucket entries of the big rows (the one-lane-per-block decoder): bucket j -> the symbol s0 holding its first slot,
    // cum[s0] and the last slots of s0, s0 + 1, s0 + 2 (4095 past the alphabet)
    for (int k = 0; k < pvc::NBIG; k++) {
        const uint16_t* row = t + pvc::SMALL_BYTES / 2 + k * pvc::BIG_ROW;
        uint64_t* ent = (uint64_t*)(out + pvc::DIRECT_OFF) + pvc::DIRECT_NB * k;
        const bool empty = row[pvc::BIG_ALPHA] == 0;
        int sym = 0;
        for (int j = 0; j < pvc::DIRECT_NB; j++) {
            const int first = pvc::DIRECT_W * j;
            while (sym < pvc::BIG_ALPHA - 1 && row[sym + 1] <= first) sym++;
            if (empty) { ent[j] = pvc::DIRECT_NONE; continue; }
            uint64_t e = (uint64_t)sym | (uint64_t)row[sym] << 7;
            for (int i = 1; i <= 3; i++) {
                const uint32_t last = sym + i <= pvc::BIG_ALPHA ? (uint32_t)row[sym + i] - 1 : (uint32_t)pvc::M - 1;
                e |= (uint64_t)(last & 0xFFF) << (7 + 12 * i);
            }
            ent[j] = e;
        }
    }
    // literal pairs (the vector decoder's two-literal step): from the LIT2 rows just written
    uint32_t* pr = (uint32_t*)(out + pvc::PAIR_OFF);
    const uint16_t* l2 = t + pvc::row_of(pvc::C_LIT2);
    for (int r = 0; r < 16; r++)
        for (int l = 0; l < 16; l++) {
            const int s1 = l >> 2, s2 = l & 3, r1 = (r & 3) * 4 + s1;
            const uint16_t* a = l2 + r * pvc::SMALL_ROW; const uint16_t* b = l2 + r1 * pvc::SMALL_ROW;
            pr[2 * (16 * r + l)] = a[s1] | (uint32_t)(a[s1 + 1] - a[s1] - pvc::M) << 16;
            pr[2 * (16 * r + l) + 1] = b[s2] | (uint32_t)(b[s2 + 1] - b[s2] - pvc::M) << 16;
        }
}

}  // namespace

struct pv_cohort {
    std::string ref_path; uint8_t ref_sha[32]; uint64_t ref_n = 0; uint32_t Q = 0; int threads = 0; int32_t form = 0;
    std::vector<std::unique_ptr<Archive>> A;
    std::vector<uint8_t> ref;                                   // REF (upper case); empty in the packed form
    std::vector<uint8_t> P, TAB;
    std::vector<uint32_t> OFF, RUN0;                            // empty in the compact-block form
    std::vector<int64_t> ST, ASM, LOW_S, LOW_L, CTG_ASM, CTG_LOCAL, CTG_BOFF, CTG_LEN;
    // packed reference form
    std::vector<uint32_t> PW, PEIX;
    std::vector<int64_t> PES, PEL;
    std::vector<uint8_t> PEB;
    // compact block-table form
    std::vector<int64_t> GRP_OFF, GRP_ST, EXC_B, EXC_ST;
    std::vector<uint16_t> BLEN;
    std::vector<int16_t> BCODE;
    std::vector<uint32_t> RUN0G;
    bool released[PV_ARR_COUNT] = {};
};

namespace {

void set_err(char* err, size_t cap, const std::string& m) {
    if (!err || !cap) return;
    const size_t k = std::min(cap - 1, m.size()); memcpy(err, m.data(), k); err[k] = 0;
}

// Compact block table of one archive (no reference layout is implied: this form is this build's own): per group of
// PV_GROUP blocks the payload offset (relative to the archive), start diagonal and first case run of its first block;
// per block a u16 payload length and an i16 code, 2 x (c - predicted c) + strand with the prediction of the format
// (previous c +- Q), or PV_CODE_EXC when the difference needs more than 15 bits: the diagonal is then looked up in
// the sorted (pooled block index, diagonal) exception table. The same information as the reference's opt-in
// CompactTab (csrc/pv_compact.h:31-49) and the same refusal of payloads over 65535 bytes (csrc/pv_core.cpp:104).
void compact_blocks(const Archive& X, const std::vector<uint32_t>& run0, uint64_t bb, uint64_t g0, pv_cohort& C,
                    std::vector<int64_t>& exc_b, std::vector<int64_t>& exc_st) {
    for (uint64_t b = 0; b < X.nb; b++) {
        const uint32_t len = X.off[b + 1] - X.off[b];
        if (len > 65535) throw FormatErr(X.path + ": block payload over 65535 B - open without compact_blocks");
        C.BLEN[bb + b] = (uint16_t)len;
        if (b % PV_GROUP == 0) {
            const uint64_t g = g0 + b / PV_GROUP;
            C.GRP_OFF[g] = X.off[b]; C.GRP_ST[g] = X.st[b]; C.RUN0G[g] = run0[b]; C.BCODE[bb + b] = 0;
            continue;
        }
        const int64_t pc = X.st[b - 1] >> 1, pred = (X.st[b - 1] & 1) ? pc - (int64_t)X.Q : pc + (int64_t)X.Q;
        const int64_t d = (X.st[b] >> 1) - pred;
        if (d >= -16383 && d <= 16383) C.BCODE[bb + b] = (int16_t)(d * 2 + (X.st[b] & 1));
        else { C.BCODE[bb + b] = PV_CODE_EXC; exc_b.push_back((int64_t)(bb + b)); exc_st.push_back(X.st[b]); }
    }
}

// The reference in 2 bits per base (A 0, C 1, G 2, T 3; base q in bits 2 (q % 16) of word q / 16) plus the maximal
// runs of any other byte as (start, length, byte), sorted, and a bucket index: for every 2^16 bases, the first run
// that ends after the bucket's start. An index gives back the byte of the plain array (reference csrc/pv_compact.h:20-29
// holds the same information; the bucket index is this build's, so a kernel finds a span's runs without a search).
void pack_reference(pv_cohort& C) {
    const uint8_t* R = C.ref.data(); const uint64_t n = C.ref_n, nw = (n + 15) / 16;
    C.PW.assign(nw + 1, 0);
    const uint64_t CH = 1u << 22;                                  // bases per chunk (a multiple of 16)
    const uint64_t nch = (n + CH - 1) / CH;
    std::vector<std::vector<int64_t>> rs(nch), rl(nch); std::vector<std::vector<uint8_t>> rb(nch);
    parallel_for(nch, C.threads, [&](uint64_t k) {
        const uint64_t q0 = k * CH, q1 = std::min(n, q0 + CH);
        for (uint64_t q = q0; q < q1;) {
            const uint8_t c = R[q];
            const int v = c == 'A' ? 0 : c == 'C' ? 1 : c == 'G' ? 2 : c == 'T' ? 3 : -1;
            if (v >= 0) { C.PW[q >> 4] |= (uint32_t)v << (2 * (q & 15)); q++; continue; }
            uint64_t e = q; while (e < q1 && R[e] == c) e++;
            rs[k].push_back((int64_t)q); rl[k].push_back((int64_t)(e - q)); rb[k].push_back(c); q = e;
        }
    });
    for (uint64_t k = 0; k < nch; k++)                          // join runs cut at chunk edges
        for (size_t j = 0; j < rs[k].size(); j++) {
            if (!C.PES.empty() && C.PES.back() + C.PEL.back() == rs[k][j] && C.PEB.back() == rb[k][j]) { C.PEL.back() += rl[k][j]; continue; }
            C.PES.push_back(rs[k][j]); C.PEL.push_back(rl[k][j]); C.PEB.push_back(rb[k][j]);
        }
    const uint64_t nbk = (n >> PV_EXC_BUCKET_BITS) + 2;
    C.PEIX.assign(nbk, 0);
    size_t r = 0;
    for (uint64_t k = 0; k < nbk; k++) {
        const uint64_t q = k << PV_EXC_BUCKET_BITS;
        while (r < C.PES.size() && (uint64_t)(C.PES[r] + C.PEL[r]) <= q) r++;
        C.PEIX[k] = (uint32_t)r;
    }
    std::vector<uint8_t>().swap(C.ref);
}

void pool(pv_cohort& C) {
    const int64_t n = (int64_t)C.A.size();
    const bool compact = C.form & PV_FORM_COMPACT_BLOCKS;
    uint64_t sp = 0, sb = 0, sl = 0, sc = 0, sg = 0;
    std::vector<uint64_t> pb(n), bb(n), lb(n), cb(n), gb(n);
    for (int64_t i = 0; i < n; i++) {
        const Archive& X = *C.A[i];
        pb[i] = sp; bb[i] = sb; lb[i] = sl; cb[i] = sc; gb[i] = sg;
        sp += X.payload_bytes; sb += X.nb + 1; sl += X.low_s.size(); sc += X.rec.size(); sg += (X.nb + PV_GROUP - 1) / PV_GROUP;
    }
    C.P.assign(sp + 64, 0);
    if (compact) {
        C.BLEN.assign(sb, 0); C.BCODE.assign(sb, 0);
        C.GRP_OFF.assign(std::max<uint64_t>(sg, 1), 0); C.GRP_ST.assign(std::max<uint64_t>(sg, 1), 0); C.RUN0G.assign(std::max<uint64_t>(sg, 1), 0);
    } else {
        C.OFF.resize(sb); C.ST.resize(sb); C.RUN0.resize(sb);
    }
    C.TAB.assign((size_t)n * pvc::GTAB_BYTES, 0); C.ASM.assign((size_t)n * 8, 0);
    C.LOW_S.resize(sl); C.LOW_L.resize(sl);
    C.CTG_ASM.resize(sc); C.CTG_LOCAL.resize(sc); C.CTG_BOFF.resize(sc); C.CTG_LEN.resize(sc);
    std::vector<std::vector<int64_t>> exb(n), exs(n);
    std::mutex mu; std::string first;
    parallel_for((uint64_t)n, C.threads, [&](uint64_t i) {
        Archive& X = *C.A[i];
        if (X.payload_bytes) memcpy(&C.P[pb[i]], X.payload.data(), X.payload_bytes);
        // first lower-case run ending after the block start
        std::vector<uint32_t> run0(X.nb + 1);
        size_t r = 0;
        for (uint64_t b = 0; b <= X.nb; b++) {
            const uint64_t bs = b * X.Q;
            while (r < X.low_s.size() && (uint64_t)(X.low_s[r] + X.low_l[r]) <= bs) r++;
            run0[b] = (uint32_t)r;
        }
        if (compact) {
            try { compact_blocks(X, run0, bb[i], gb[i], C, exb[i], exs[i]); }
            catch (const FormatErr& e) { std::lock_guard<std::mutex> g(mu); if (first.empty()) first = e.what(); }
        } else {
            memcpy(&C.OFF[bb[i]], X.off.data(), (X.nb + 1) * 4);
            memcpy(&C.ST[bb[i]], X.st.data(), (X.nb + 1) * 8);
            memcpy(&C.RUN0[bb[i]], run0.data(), (X.nb + 1) * 4);
        }
        build_gtab(X, &C.TAB[(size_t)i * pvc::GTAB_BYTES]);
        int64_t* q = &C.ASM[(size_t)i * 8];
        q[0] = (int64_t)pb[i]; q[1] = (int64_t)bb[i]; q[2] = (int64_t)X.nbases; q[3] = (int64_t)lb[i]; q[4] = (int64_t)X.low_s.size();
        q[5] = (int64_t)gb[i];
        if (!X.low_s.empty()) { memcpy(&C.LOW_S[lb[i]], X.low_s.data(), X.low_s.size() * 8); memcpy(&C.LOW_L[lb[i]], X.low_l.data(), X.low_l.size() * 8); }
        for (size_t r2 = 0; r2 < X.rec.size(); r2++) {
            const uint64_t k = cb[i] + r2;
            C.CTG_ASM[k] = (int64_t)i; C.CTG_LOCAL[k] = (int64_t)r2; C.CTG_BOFF[k] = (int64_t)X.rec[r2].boff; C.CTG_LEN[k] = (int64_t)X.rec[r2].len;
        }
        // the archive's own copies are no longer needed (runs stay: fasta / case application use them)
        std::vector<uint8_t>().swap(X.payload); std::vector<uint32_t>().swap(X.off); std::vector<int64_t>().swap(X.st);
    });
    if (!first.empty()) throw FormatErr(first);
    for (int64_t i = 0; i < n; i++) {                          // pooled block index order: archive by archive
        C.EXC_B.insert(C.EXC_B.end(), exb[i].begin(), exb[i].end());
        C.EXC_ST.insert(C.EXC_ST.end(), exs[i].begin(), exs[i].end());
    }
    if (C.form & PV_FORM_PACKED_REF) pack_reference(C);
}

const Archive* archive_at(const pv_cohort* c, int64_t a) {
    if (!c || a < 0 || a >= (int64_t)c->A.size()) return nullptr;
    return c->A[(size_t)a].get();
}

uint64_t fasta_bytes(const Archive& X) {
    uint64_t size = 0;
    for (auto& r : X.rec) size += 2 + r.hdr.size() + r.len + (r.lw ? (r.len + r.lw - 1) / r.lw : 0);
    return size;
}

}  // namespace

extern "C" {

int32_t pv_abi_version(void) { return PV_ABI_VERSION; }

int32_t pv_cohort_open(const char* reference, const char* const* paths, int32_t npaths, int32_t threads, int32_t form,
                       pv_cohort** out, char* err, size_t errcap) {
    if (out) *out = nullptr;
    if (!reference || !paths || !out) { set_err(err, errcap, "null argument"); return PV_EARG; }
    if (form & ~(PV_FORM_PACKED_REF | PV_FORM_COMPACT_BLOCKS)) { set_err(err, errcap, "unknown form bits"); return PV_EARG; }
    try {
        if (npaths <= 0) throw FormatErr("no archives");
        std::unique_ptr<pv_cohort> C(new pv_cohort());
        C->ref_path = reference; C->threads = threads > 0 ? threads : host_threads(); C->form = form;
        C->ref = read_file(reference);
        C->ref_n = fasta_to_bases(C->ref.data(), C->ref.size(), reference);
        C->ref.resize(C->ref_n); C->ref.shrink_to_fit();
        pvs::sha256(C->ref.data(), C->ref_n, C->ref_sha);
        if (C->ref_n >= (1ull << 32)) throw FormatErr("reference of 2^32 bases or more: copy positions are 32-bit");
        C->A.resize((size_t)npaths);
        std::mutex mu; std::string first; bool first_is_format = true;
        parallel_for((uint64_t)npaths, C->threads, [&](uint64_t i) {
            try {
                const std::vector<uint8_t> f = read_file(paths[i]);
                std::unique_ptr<Archive> X(new Archive());
                open_archive(f, paths[i], C->ref_sha, C->ref_n, *X);
                C->A[i] = std::move(X);
            } catch (const FormatErr& e) {
                std::lock_guard<std::mutex> g(mu); if (first.empty()) first = e.what();
            } catch (const std::exception& e) {
                std::lock_guard<std::mutex> g(mu); if (first.empty()) { first = e.what(); first_is_format = false; }
            }
        });
        if (!first.empty()) { if (first_is_format) throw FormatErr(first); throw std::runtime_error(first); }
        C->Q = C->A[0]->Q;
        for (auto& x : C->A)
            if (x->Q != C->Q)
                throw FormatErr(x->path + ": block size " + std::to_string(x->Q) + " differs from " + std::to_string(C->Q) + " (one dataset per cohort)");
        pool(*C);
        *out = C.release();
        return PV_OK;
    } catch (const FormatErr& e) { set_err(err, errcap, e.what()); return PV_EFORMAT; }
    catch (const std::bad_alloc&) { set_err(err, errcap, "out of host memory"); return PV_ENOMEM; }
    catch (const std::exception& e) { set_err(err, errcap, e.what()); return PV_EARG; }
}

void pv_cohort_close(pv_cohort* c) { delete c; }

int32_t pv_cohort_block_size(const pv_cohort* c) { return c ? (int32_t)c->Q : 0; }
int64_t pv_cohort_assemblies(const pv_cohort* c) { return c ? (int64_t)c->A.size() : 0; }
uint64_t pv_cohort_ref_bases(const pv_cohort* c) { return c ? c->ref_n : 0; }
void pv_cohort_ref_sha256(const pv_cohort* c, char out_hex[65]) {
    if (!c || !out_hex) return;
    const std::string h = hex(c->ref_sha, 32); memcpy(out_hex, h.c_str(), 65);
}

int32_t pv_cohort_array(const pv_cohort* c, int32_t id, const void** ptr, uint64_t* nbytes) {
    if (!c || !ptr || !nbytes || id < 0 || id >= PV_ARR_COUNT) return PV_EARG;
    if (c->released[id]) { *ptr = nullptr; *nbytes = 0; return PV_EARG; }
    switch (id) {
        case PV_ARR_P: *ptr = c->P.data(); *nbytes = c->P.size(); break;
        case PV_ARR_OFF: *ptr = c->OFF.data(); *nbytes = c->OFF.size() * 4; break;
        case PV_ARR_ST: *ptr = c->ST.data(); *nbytes = c->ST.size() * 8; break;
        case PV_ARR_RUN0: *ptr = c->RUN0.data(); *nbytes = c->RUN0.size() * 4; break;
        case PV_ARR_TAB: *ptr = c->TAB.data(); *nbytes = c->TAB.size(); break;
        case PV_ARR_ASM: *ptr = c->ASM.data(); *nbytes = c->ASM.size() * 8; break;
        case PV_ARR_LOW_S: *ptr = c->LOW_S.data(); *nbytes = c->LOW_S.size() * 8; break;
        case PV_ARR_LOW_L: *ptr = c->LOW_L.data(); *nbytes = c->LOW_L.size() * 8; break;
        case PV_ARR_REF: *ptr = c->ref.data(); *nbytes = c->ref.size(); break;
        case PV_ARR_CTG_ASM: *ptr = c->CTG_ASM.data(); *nbytes = c->CTG_ASM.size() * 8; break;
        case PV_ARR_CTG_LOCAL: *ptr = c->CTG_LOCAL.data(); *nbytes = c->CTG_LOCAL.size() * 8; break;
        case PV_ARR_CTG_BOFF: *ptr = c->CTG_BOFF.data(); *nbytes = c->CTG_BOFF.size() * 8; break;
        case PV_ARR_CTG_LEN: *ptr = c->CTG_LEN.data(); *nbytes = c->CTG_LEN.size() * 8; break;
        case PV_ARR_PW: *ptr = c->PW.data(); *nbytes = c->PW.size() * 4; break;
        case PV_ARR_PES: *ptr = c->PES.data(); *nbytes = c->PES.size() * 8; break;
        case PV_ARR_PEL: *ptr = c->PEL.data(); *nbytes = c->PEL.size() * 8; break;
        case PV_ARR_PEB: *ptr = c->PEB.data(); *nbytes = c->PEB.size(); break;
        case PV_ARR_PEIX: *ptr = c->PEIX.data(); *nbytes = c->PEIX.size() * 4; break;
        case PV_ARR_GRP_OFF: *ptr = c->GRP_OFF.data(); *nbytes = c->GRP_OFF.size() * 8; break;
        case PV_ARR_GRP_ST: *ptr = c->GRP_ST.data(); *nbytes = c->GRP_ST.size() * 8; break;
        case PV_ARR_RUN0G: *ptr = c->RUN0G.data(); *nbytes = c->RUN0G.size() * 4; break;
        case PV_ARR_BLEN: *ptr = c->BLEN.data(); *nbytes = c->BLEN.size() * 2; break;
        case PV_ARR_BCODE: *ptr = c->BCODE.data(); *nbytes = c->BCODE.size() * 2; break;
        case PV_ARR_EXC_B: *ptr = c->EXC_B.data(); *nbytes = c->EXC_B.size() * 8; break;
        case PV_ARR_EXC_ST: *ptr = c->EXC_ST.data(); *nbytes = c->EXC_ST.size() * 8; break;
        default: return PV_EARG;
    }
    return PV_OK;
}

int32_t pv_cohort_form(const pv_cohort* c) { return c ? c->form : 0; }
int64_t pv_cohort_ref_exceptions(const pv_cohort* c) { return c ? (int64_t)c->PES.size() : 0; }
int64_t pv_cohort_block_exceptions(const pv_cohort* c) { return c ? (int64_t)c->EXC_B.size() : 0; }

int32_t pv_cohort_release_array(pv_cohort* c, int32_t id) {
    if (!c || id < 0 || id >= PV_ARR_COUNT) return PV_EARG;
    switch (id) {
        case PV_ARR_P: std::vector<uint8_t>().swap(c->P); break;
        case PV_ARR_OFF: std::vector<uint32_t>().swap(c->OFF); break;
        case PV_ARR_ST: std::vector<int64_t>().swap(c->ST); break;
        case PV_ARR_RUN0: std::vector<uint32_t>().swap(c->RUN0); break;
        case PV_ARR_TAB: std::vector<uint8_t>().swap(c->TAB); break;
        case PV_ARR_REF: std::vector<uint8_t>().swap(c->ref); break;
        case PV_ARR_PW: std::vector<uint32_t>().swap(c->PW); break;
        case PV_ARR_BLEN: std::vector<uint16_t>().swap(c->BLEN); break;
        case PV_ARR_BCODE: std::vector<int16_t>().swap(c->BCODE); break;
        case PV_ARR_GRP_OFF: std::vector<int64_t>().swap(c->GRP_OFF); break;
        case PV_ARR_GRP_ST: std::vector<int64_t>().swap(c->GRP_ST); break;
        case PV_ARR_RUN0G: std::vector<uint32_t>().swap(c->RUN0G); break;
        default: return PV_EARG;   // small tables and the case runs stay on the host (fasta, case application)
    }
    c->released[id] = true;
    return PV_OK;
}

int32_t pv_asm_info_get(const pv_cohort* c, int64_t a, pv_asm_info* out) {
    const Archive* X = archive_at(c, a);
    if (!X || !out) return PV_EARG;
    memset(out, 0, sizeof *out);
    out->Q = X->Q; out->flags = X->flags; out->bases = X->nbases; out->blocks = X->nb; out->file_bytes = X->file_bytes;
    out->payload_bytes = X->payload_bytes; out->contigs = X->rec.size(); out->lower_case_runs = X->low_s.size();
    out->fasta_xxh3 = X->fasta_xxh; out->bases_xxh3 = X->bases_xxh; out->block_hashes = !X->hashes.empty();
    snprintf(out->path, sizeof out->path, "%s", X->path.c_str());
    snprintf(out->reference_name, sizeof out->reference_name, "%s", X->refname.c_str());
    return PV_OK;
}

int32_t pv_asm_contig(const pv_cohort* c, int64_t a, int64_t k, const char** name, const char** header, uint64_t* length,
                      uint64_t* offset, uint32_t* line_width) {
    const Archive* X = archive_at(c, a);
    if (!X || k < 0 || k >= (int64_t)X->rec.size()) return PV_EARG;
    const Contig& r = X->rec[(size_t)k];
    if (name) *name = r.name.c_str();
    if (header) *header = r.hdr.c_str();
    if (length) *length = r.len;
    if (offset) *offset = r.boff;
    if (line_width) *line_width = r.lw;
    return PV_OK;
}

int32_t pv_fasta_xxh3(const pv_cohort* c, int64_t a, const uint8_t* bases, uint64_t n, uint64_t* hash, char* err, size_t errcap) {
    const Archive* X = archive_at(c, a);
    if (!X || !hash || (!bases && n)) { set_err(err, errcap, "bad arguments"); return PV_EARG; }
    if (n != X->nbases) { set_err(err, errcap, "bases: uint8 CPU tensor of the assembly's length"); return PV_EFORMAT; }
    // the file is streamed through a 1 MiB staging buffer: header, then lines copied with their line end; lines of
    // 4 KiB or more go to the hash straight from `bases`
    pvx::Stream h;
    const size_t CAP = 1u << 20;
    std::unique_ptr<uint8_t[]> buf(new uint8_t[CAP + 8]);
    size_t used = 0;
    auto drain = [&]() { h.update(buf.get(), used); used = 0; };
    for (auto& r : X->rec) {
        if (used + r.hdr.size() + 2 > CAP) drain();
        if (r.hdr.size() + 2 > CAP) {
            const uint8_t gt = '>', nl = '\n';
            h.update(&gt, 1); h.update(r.hdr.data(), r.hdr.size()); h.update(&nl, 1);
        } else {
            buf[used++] = '>'; memcpy(buf.get() + used, r.hdr.data(), r.hdr.size()); used += r.hdr.size(); buf[used++] = '\n';
        }
        const uint8_t* src = bases + r.boff;
        for (uint64_t x = 0; x < r.len; x += r.lw) {
            const uint64_t k = std::min<uint64_t>(r.lw, r.len - x);
            if (k >= 4096) {
                drain(); h.update(src + x, k); buf[used++] = '\n';
                continue;
            }
            if (used + k + 1 > CAP) drain();
            memcpy(buf.get() + used, src + x, k); used += k; buf[used++] = '\n';
        }
    }
    drain();
    *hash = h.digest();
    return PV_OK;
}

uint64_t pv_fasta_size(const pv_cohort* c, int64_t a) { const Archive* X = archive_at(c, a); return X ? fasta_bytes(*X) : 0; }

int32_t pv_fasta_build(const pv_cohort* c, int64_t a, const uint8_t* bases, uint64_t n, uint8_t* out, uint64_t cap, char* err, size_t errcap) {
    const Archive* X = archive_at(c, a);
    if (!X || !out || (!bases && n)) { set_err(err, errcap, "bad arguments"); return PV_EARG; }
    if (n != X->nbases || cap < fasta_bytes(*X)) { set_err(err, errcap, "FASTA size"); return PV_EARG; }
    uint8_t* p = out;
    for (auto& r : X->rec) {
        *p++ = '>'; memcpy(p, r.hdr.data(), r.hdr.size()); p += r.hdr.size(); *p++ = '\n';
        for (uint64_t x = 0; x < r.len; x += r.lw) {
            const uint64_t k = std::min<uint64_t>(r.lw, r.len - x);
            memcpy(p, bases + r.boff + x, k); p += k; *p++ = '\n';
        }
    }
    return PV_OK;
}

int32_t pv_verify_blocks(const pv_cohort* c, int64_t a, const uint8_t* upper, uint64_t n, int64_t* first_bad) {
    const Archive* X = archive_at(c, a);
    if (!X || !first_bad || n != X->nbases || (!upper && n)) return PV_EARG;
    *first_bad = -1;
    if (X->hashes.empty()) return PV_OK;
    std::atomic<int64_t> bad{INT64_MAX};
    const uint64_t per = 256;
    parallel_for((X->nb + per - 1) / per, c->threads, [&](uint64_t g) {
        for (uint64_t b = g * per; b < std::min(X->nb, (g + 1) * per); b++) {
            const uint64_t bs = b * X->Q, len = std::min<uint64_t>(X->Q, X->nbases - bs);
            if (pvx::xxh3_64(upper + bs, len) != X->hashes[b]) {
                int64_t cur = bad.load();
                while ((int64_t)b < cur && !bad.compare_exchange_weak(cur, (int64_t)b)) {}
            }
        }
    });
    if (bad.load() != INT64_MAX) *first_bad = bad.load();
    return PV_OK;
}

int32_t pv_apply_case(const pv_cohort* c, int64_t a, uint64_t s, uint8_t* bases, uint64_t n) {
    const Archive* X = archive_at(c, a);
    if (!X || (!bases && n) || s > X->nbases || n > X->nbases - s) return PV_EARG;
    // first run ending after s (reference csrc/pv_v1.h:160-162), then every run starting before s + n
    size_t lo = 0, hi = X->low_s.size();
    while (lo < hi) { const size_t m = (lo + hi) / 2; if ((uint64_t)(X->low_s[m] + X->low_l[m]) <= s) lo = m + 1; else hi = m; }
    for (size_t r = lo; r < X->low_s.size() && (uint64_t)X->low_s[r] < s + n; r++) {
        const uint64_t x0 = std::max<uint64_t>(s, (uint64_t)X->low_s[r]), x1 = std::min<uint64_t>(s + n, (uint64_t)(X->low_s[r] + X->low_l[r]));
        for (uint64_t x = x0; x < x1; x++) bases[x - s] |= 0x20;
    }
    return PV_OK;
}

uint64_t pv_xxh3_64(const void* data, uint64_t n) { return pvx::xxh3_64(data, n); }
uint64_t pv_xxh3_64_parts(const void* const* ptrs, const uint64_t* sizes, int32_t parts) {
    pvx::Stream h;
    for (int32_t i = 0; i < parts; i++) h.update(ptrs[i], sizes[i]);
    return h.digest();
}

// incremental XXH3-64 (seed 0) over data that arrives in pieces (the check_full pipeline hashes the FASTA chunk by
// chunk as the device produces it)
void* pv_xxh3_stream_new(void) { return new (std::nothrow) pvx::Stream(); }
void pv_xxh3_stream_update(void* h, const void* data, uint64_t n) { if (h && (data || !n)) static_cast<pvx::Stream*>(h)->update(data, n); }
uint64_t pv_xxh3_stream_digest(const void* h) { return h ? static_cast<const pvx::Stream*>(h)->digest() : 0; }
void pv_xxh3_stream_free(void* h) { delete static_cast<pvx::Stream*>(h); }

int32_t pv_sha256_file_bases(const char* path, char out_hex[65], char* err, size_t errcap) {
    if (!path || !out_hex) { set_err(err, errcap, "null argument"); return PV_EARG; }
    try {
        std::vector<uint8_t> b = read_file(path);
        const uint64_t n = fasta_to_bases(b.data(), b.size(), path);
        uint8_t s[32]; pvs::sha256(b.data(), n, s);
        const std::string h = hex(s, 32); memcpy(out_hex, h.c_str(), 65);
        return PV_OK;
    } catch (const FormatErr& e) { set_err(err, errcap, e.what()); return PV_EFORMAT; }
    catch (const std::exception& e) { set_err(err, errcap, e.what()); return PV_EARG; }
}

}  // extern "C"
