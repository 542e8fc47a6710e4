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

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cerrno>
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

// ---- bytes in

// A bounds-checked cursor over a byte span. A read that does not fit in what is left marks the cursor failed and
// returns zero, and every read after it fails too, so a parser reads a whole table and tests the cursor once.
class Cursor {
public:
    Cursor(const uint8_t* data, size_t size) : data_(data), size_(size) {}
    template <class T> T get() {
        T v{};
        if (const uint8_t* p = take(sizeof(T))) memcpy(&v, p, sizeof(T));
        return v;
    }
    // LEB128: seven bits per byte, the low group first, the high bit set on every byte but the last; ten bytes at most
    uint64_t varint() {
        uint64_t v = 0;
        for (unsigned shift = 0; shift < 64; shift += 7) {
            const uint8_t* p = take(1);
            if (!p) return 0;
            v |= (uint64_t)(*p & 0x7F) << shift;
            if (!(*p & 0x80)) return v;
        }
        failed_ = true;
        return 0;
    }
    const uint8_t* bytes(size_t n) { return take(n); }
    void fail() { failed_ = true; }
    bool ok() const { return !failed_; }
    bool at_end() const { return pos_ == size_; }
    size_t size() const { return size_; }

private:
    const uint8_t* take(size_t n) {
        if (failed_ || n > size_ - pos_) { failed_ = true; return nullptr; }
        const uint8_t* p = data_ + pos_;
        pos_ += n;
        return p;
    }
    const uint8_t* data_;
    size_t size_, pos_ = 0;
    bool failed_ = false;
};

// A whole file, by POSIX reads
std::vector<uint8_t> load_file(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw FormatErr(path + ": cannot open");
    std::vector<uint8_t> data;
    struct stat sb{};
    bool whole = ::fstat(fd, &sb) == 0 && sb.st_size >= 0;
    if (whole) {
        data.resize((size_t)sb.st_size);
        size_t got = 0;
        while (got < data.size()) {
            const ssize_t r = ::read(fd, data.data() + got, data.size() - got);
            if (r > 0) got += (size_t)r;
            else if (r < 0 && errno == EINTR) continue;
            else break;
        }
        whole = got == data.size();
    }
    ::close(fd);
    if (!whole) throw FormatErr(path + ": short read");
    return data;
}

std::string to_hex(const uint8_t* p, size_t n) {
    std::string s(2 * n, '0');
    for (size_t i = 0; i < n; i++) snprintf(&s[2 * i], 3, "%02x", p[i]);
    return s;
}

// The reference's FASTA bytes become its bases in place: lines that start with '>' and the line ends go, lower-case
// letters become upper case. Every line, the last too, ends with '\n'. Returns the base count.
uint64_t fasta_to_bases(uint8_t* buf, uint64_t size, const std::string& path) {
    static const std::array<uint8_t, 256> upper = [] {
        std::array<uint8_t, 256> t{};
        for (int c = 0; c < 256; c++) t[c] = (uint8_t)(c >= 'a' && c <= 'z' ? c - ('a' - 'A') : c);
        return t;
    }();
    if (size == 0 || buf[0] != '>') throw FormatErr(path + ": not FASTA (no header at byte 0)");
    uint64_t kept = 0;
    for (uint64_t line = 0; line < size;) {
        const uint8_t* eol = (const uint8_t*)memchr(buf + line, '\n', size - line);
        const bool header = buf[line] == '>';
        if (!eol) throw FormatErr(path + (header ? ": header without line end" : ": no final line end"));
        const uint64_t end = (uint64_t)(eol - buf);
        if (!header)                                           // the write position never passes the read position
            for (uint64_t k = line; k < end; k++) buf[kept++] = upper[buf[k]];
        line = end + 1;
    }
    return kept;
}

// f(i) for every i in [0, n) on up to `threads` threads, thread t taking i = t, t + T, t + 2T, ... (the caller's thread
// is thread 0)
template <class F> void run_parallel(uint64_t n, int threads, F&& f) {
    const uint64_t T = std::min<uint64_t>(n, (uint64_t)std::max(threads, 1));
    std::vector<std::thread> helpers;
    for (uint64_t t = 1; t < T; t++)
        helpers.emplace_back([&f, t, T, n] { for (uint64_t i = t; i < n; i += T) f(i); });
    for (uint64_t i = 0; i < n; i += std::max<uint64_t>(T, 1)) f(i);
    for (auto& h : helpers) h.join();
}
int online_cpus() { const long c = sysconf(_SC_NPROCESSORS_ONLN); return c > 0 ? (int)c : 4; }

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

// ---- the archive header (format section 1): 136 bytes at fixed offsets, then a u16 name length and the name
constexpr uint8_t kMagic[8] = {'R', 'F', 'R', 'L', '3', 'V', '1', 0};
constexpr uint32_t kVersion = 1, kBlockHashes = 1, kHeaderBytes = 136, kFixedBytes = kHeaderBytes + 2;
struct Header {
    uint8_t magic[8];                                          //   0
    uint32_t version, Q, flags, reserved;                      //   8  12  16  20
    uint8_t ref_sha[32];                                       //  24
    uint64_t ref_bases, bases, blocks, fasta_xxh3, bases_xxh3; //  56  64  72  80  88
    uint64_t meta_packed, meta_bytes, hash_bytes, payload;     //  96 104 112 120
    uint64_t header_xxh3;                                      // 128
    uint16_t name_len;                                         // 136
};
Header parse_header(const uint8_t* file) {
    Cursor c(file, kFixedBytes);
    Header h;
    memcpy(h.magic, c.bytes(8), 8);
    h.version = c.get<uint32_t>(); h.Q = c.get<uint32_t>(); h.flags = c.get<uint32_t>(); h.reserved = c.get<uint32_t>();
    memcpy(h.ref_sha, c.bytes(32), 32);
    uint64_t* wide[] = {&h.ref_bases, &h.bases, &h.blocks, &h.fasta_xxh3, &h.bases_xxh3, &h.meta_packed, &h.meta_bytes,
                        &h.hash_bytes, &h.payload, &h.header_xxh3};
    for (uint64_t* f : wide) *f = c.get<uint64_t>();
    h.name_len = c.get<uint16_t>();
    return h;
}

// What the header checks see: the file, its header, and the reference the cohort was opened with
struct Opened {
    const uint8_t* file; uint64_t size;
    Header h;
    const uint8_t* ref_sha; uint64_t ref_bases;
    uint64_t meta_at() const { return kFixedBytes + h.name_len; }
    uint64_t payload_at() const { return meta_at() + h.meta_packed + h.hash_bytes; }
};
bool sections_fit(const Opened& o) {        // name, meta, hashes and payload tile the file after the header
    const uint64_t parts[] = {o.meta_at(), o.h.meta_packed, o.h.hash_bytes, o.h.payload};
    uint64_t sum = 0;
    for (uint64_t p : parts) {
        if (p > o.size) return false;
        sum += p;
    }
    return sum == o.size;
}
bool header_hash_matches(const Opened& o) { // XXH3 of [0, payload) with the hash field read as zero
    static const uint8_t zero[8] = {};
    pvx::Stream s;
    s.update(o.file, 128); s.update(zero, 8); s.update(o.file + kHeaderBytes, o.payload_at() - kHeaderBytes);
    return s.digest() == o.h.header_xxh3;
}
// The header's checks in the format's order (section 5), each with its refusal
struct HeaderRule { const char* refusal; bool (*holds)(const Opened&); };
const HeaderRule kHeaderRules[] = {
    {"magic (not refrel3 v1)", [](const Opened& o) { return memcmp(o.h.magic, kMagic, 8) == 0; }},
    {"version", [](const Opened& o) { return o.h.version == kVersion; }},
    {"block size", [](const Opened& o) { return o.h.Q == 1024 || o.h.Q == 2048 || o.h.Q == 4096 || o.h.Q == 16384; }},
    {"unknown flags", [](const Opened& o) { return (o.h.flags & ~kBlockHashes) == 0; }},
    {"reserved", [](const Opened& o) { return o.h.reserved == 0; }},
    {"section sizes", sections_fit},
    {"block count", [](const Opened& o) { return o.h.blocks == o.h.bases / o.h.Q + (o.h.bases % o.h.Q != 0); }},
    {"hash section size", [](const Opened& o) {
         return (o.h.flags & kBlockHashes) ? o.h.blocks <= o.size / 8 && o.h.hash_bytes == 8 * o.h.blocks : o.h.hash_bytes == 0; }},
    {"header XXH3", header_hash_matches},
    {"reference SHA-256 / size differs (wrong reference)", [](const Opened& o) {
         return memcmp(o.h.ref_sha, o.ref_sha, 32) == 0 && o.h.ref_bases == o.ref_bases; }},
};

// ---- the meta section (format section 2), table by table: each returns its refusal, or nullptr

// 2.1 the contig table: u32 count; per record a u32-prefixed header line, u64 length, u32 line width
const char* read_contigs(Cursor& m, Archive& X) {
    const uint32_t count = m.get<uint32_t>();
    if (count > m.size()) return "records";
    X.rec.reserve(count);
    uint64_t at = 0;
    for (uint32_t k = 0; k < count && m.ok(); k++) {
        Contig r;
        const uint32_t hl = m.get<uint32_t>();
        const uint8_t* line = m.bytes(hl);
        if (!line) break;
        r.hdr.assign((const char*)line, hl);
        r.len = m.get<uint64_t>();
        r.lw = m.get<uint32_t>();
        if (r.len && !r.lw) m.fail();
        r.name = r.hdr.substr(0, r.hdr.find_first_of(" \t"));
        r.boff = at;
        at += r.len;
        X.rec.push_back(std::move(r));
    }
    return m.ok() && at == X.nbases ? nullptr : "contig table";
}
// 2.2 lower-case runs: u64 count; per run LEB128 gap after the previous run, LEB128 length, inside the assembly
const char* read_case_runs(Cursor& m, Archive& X) {
    const uint64_t count = m.get<uint64_t>();
    if (count > X.nbases) return "case runs";
    const uint64_t room = std::min<uint64_t>(count, m.size() / 2);    // each run takes two bytes at least
    X.low_s.reserve(room); X.low_l.reserve(room);
    uint64_t end = 0;
    for (uint64_t k = 0; k < count && m.ok(); k++) {
        const uint64_t gap = m.varint(), len = m.varint();
        if (gap > X.nbases - end || len > X.nbases - end - gap) { m.fail(); break; }
        X.low_s.push_back((int64_t)(end + gap));
        X.low_l.push_back((int64_t)len);
        end += gap + len;
    }
    return m.ok() ? nullptr : "case runs";
}
// 2.3 model tables: per context, a LEB128 frequency per symbol; a context sums to the probability scale or is empty
const char* read_models(Cursor& m, Archive& X) {
    X.freq.assign((size_t)pvc::NCTX * pvc::BIG_ALPHA, 0);
    for (int c = 0; c < pvc::NCTX; c++) {
        uint16_t* row = &X.freq[(size_t)c * pvc::BIG_ALPHA];
        uint64_t total = 0;
        for (int s = 0; s < pvc::alpha_of(c); s++) {
            const uint64_t f = m.varint();
            if (f > pvc::M) m.fail();
            row[s] = (uint16_t)f;
            total += f;
        }
        if (total && total != pvc::M) m.fail();
        if (!m.ok()) return "model tables";
    }
    return nullptr;
}
// 2.4 the block table: per block a LEB128 payload length and a LEB128 start code, zigzag(c - expected) * 2 + strand,
// where block b's expected diagonal is block b - 1's moved one block along its strand (0 for block 0); the lengths sum
// to the payload and nothing follows the table
const char* read_block_table(Cursor& m, Archive& X, uint64_t payload) {
    if (X.nb > m.size() / 2) return "block table";              // each block takes two bytes at least
    X.off.assign(X.nb + 1, 0);
    X.st.assign(X.nb + 1, 0);
    uint64_t used = 0;
    int64_t diag = 0;
    uint32_t strand = 0;
    for (uint64_t b = 0; b < X.nb && m.ok(); b++) {
        const uint64_t len = m.varint();
        if (len > payload - used) { m.fail(); break; }
        used += len;
        X.off[b + 1] = (uint32_t)used;
        const uint64_t code = m.varint();
        const int64_t expected = b == 0 ? 0 : strand ? diag - (int64_t)X.Q : diag + (int64_t)X.Q;
        diag = (int64_t)((uint64_t)expected + (uint64_t)pvc::unzigzag(code >> 1));
        strand = (uint32_t)(code & 1);
        X.st[b] = (int64_t)(((uint64_t)diag << 1) | strand);
    }
    return m.ok() && m.at_end() && used == payload ? nullptr : "block table";
}

// One archive, every check of the format before any decode, refused with "<path>: refused: <why>"
void open_archive(const std::vector<uint8_t>& file, const std::string& path, const uint8_t ref_sha[32], uint64_t ref_bases, Archive& X) {
    auto refuse = [&](const char* why) { throw FormatErr(path + ": refused: " + why); };
    if (file.size() < kFixedBytes) refuse("short file");
    const Opened o{file.data(), file.size(), parse_header(file.data()), ref_sha, ref_bases};
    for (const HeaderRule& r : kHeaderRules)
        if (!r.holds(o)) refuse(r.refusal);
    X.Q = o.h.Q; X.flags = o.h.flags; X.nbases = o.h.bases; X.nb = o.h.blocks;
    X.fasta_xxh = o.h.fasta_xxh3; X.bases_xxh = o.h.bases_xxh3;
    X.refname.assign((const char*)file.data() + kFixedBytes, o.h.name_len);
    // the meta section: exactly one zstd frame of the stated decompressed size
    const uint8_t* packed = file.data() + o.meta_at();
    if (o.h.meta_bytes > (1ull << 32) || ZSTD_getFrameContentSize(packed, o.h.meta_packed) != o.h.meta_bytes) refuse("meta frame");
    if (ZSTD_findFrameCompressedSize(packed, o.h.meta_packed) != o.h.meta_packed) refuse("meta frame count (exactly one zstd frame)");
    std::vector<uint8_t> meta(o.h.meta_bytes);
    if (ZSTD_decompress(meta.data(), meta.size(), packed, o.h.meta_packed) != meta.size()) refuse("meta decompress");
    Cursor m(meta.data(), meta.size());
    if (const char* why = read_contigs(m, X)) refuse(why);
    if (const char* why = read_case_runs(m, X)) refuse(why);
    if (const char* why = read_models(m, X)) refuse(why);
    if (o.h.payload >= (1ull << 32)) refuse("payload over 4 GiB (pooled offsets are 32-bit)");
    if (const char* why = read_block_table(m, X, o.h.payload)) refuse(why);
    if (X.flags & kBlockHashes) {
        X.hashes.resize(X.nb);
        memcpy(X.hashes.data(), packed + o.h.meta_packed, X.nb * 8);
    }
    X.payload.assign(file.begin() + (ptrdiff_t)o.payload_at(), file.end());
    X.payload_bytes = o.h.payload; X.file_bytes = file.size(); X.path = path;
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

// ---- the compact block-table form (this build's own layout): per group of PV_GROUP blocks the payload offset, start
// diagonal and first case run of its first block; per block a u16 payload length and an i16 step code. The same
// information as the reference's opt-in CompactTab (csrc/pv_compact.h:31-49), with the same refusal of payloads over
// 65535 bytes (csrc/pv_core.cpp:104).

// Block b's step code from block b - 1's start and its own: 2 x (c - the expected c) + strand, the expectation being the
// format's (block b - 1's diagonal moved one block along its strand); PV_CODE_EXC where that does not fit in an i16
// other than PV_CODE_EXC itself (the start then goes to the exception table).
int16_t step_code(int64_t prev, int64_t cur, uint32_t Q) {
    const int64_t expected = (prev >> 1) + ((prev & 1) ? -(int64_t)Q : (int64_t)Q);
    const int64_t code = 2 * ((cur >> 1) - expected) + (cur & 1);
    return code > PV_CODE_EXC && code <= INT16_MAX ? (int16_t)code : (int16_t)PV_CODE_EXC;
}

// Per-archive placement in the pooled arrays: where its payload bytes, block rows (blocks + 1), case runs, contigs and
// block groups begin
struct Placement { uint64_t payload = 0, blocks = 0, runs = 0, contigs = 0, groups = 0; };

// For each block start (and the stream's end), the first case run that ends after it
std::vector<uint32_t> first_runs(const Archive& X) {
    std::vector<int64_t> ends(X.low_s.size());
    for (size_t r = 0; r < ends.size(); r++) ends[r] = X.low_s[r] + X.low_l[r];
    std::vector<uint32_t> out(X.nb + 1);
    for (uint64_t b = 0; b <= X.nb; b++)
        out[b] = (uint32_t)(std::upper_bound(ends.begin(), ends.end(), (int64_t)(b * X.Q)) - ends.begin());
    return out;
}

// One archive's rows of the compact table; starts that need the exception table are appended to `exc` as (pooled
// block, start)
void place_compact(const Archive& X, const std::vector<uint32_t>& run0, const Placement& at, pv_cohort& C,
                   std::vector<std::pair<int64_t, int64_t>>& exc) {
    for (uint64_t b = 0; b < X.nb; b++) {
        const uint64_t row = at.blocks + b;
        const uint32_t len = X.off[b + 1] - X.off[b];
        if (len > UINT16_MAX) throw FormatErr(X.path + ": block payload over 65535 B - open without compact_blocks");
        C.BLEN[row] = (uint16_t)len;
        if (b % PV_GROUP == 0) {                                // a group's first block: absolute offset and start
            const uint64_t g = at.groups + b / PV_GROUP;
            C.GRP_OFF[g] = X.off[b]; C.GRP_ST[g] = X.st[b]; C.RUN0G[g] = run0[b];
            C.BCODE[row] = 0;
            continue;
        }
        C.BCODE[row] = step_code(X.st[b - 1], X.st[b], X.Q);
        if (C.BCODE[row] == PV_CODE_EXC) exc.emplace_back((int64_t)row, X.st[b]);
    }
}

// ---- the packed reference form: 2 bits per base (A 0, C 1, G 2, T 3; base q in bits 2 (q % 16) of word q / 16), the
// maximal runs of any other byte as (start, length, byte) in order, and a bucket index - per 2^PV_EXC_BUCKET_BITS
// bases, the first run that ends after the bucket's start - so that a kernel finds a span's runs without a search.
// The reference's csrc/pv_compact.h:20-29 holds the same information in its own layout.
struct ByteRun { uint64_t start, end; uint8_t byte; };

void pack_reference(pv_cohort& C) {
    static const std::array<uint8_t, 256> code = [] {
        std::array<uint8_t, 256> t;
        t.fill(4);
        t['A'] = 0; t['C'] = 1; t['G'] = 2; t['T'] = 3;
        return t;
    }();
    const uint8_t* R = C.ref.data();
    const uint64_t n = C.ref_n;
    C.PW.assign((n + 15) / 16 + 1, 0);
    constexpr uint64_t SPAN = 1ull << 22;                      // bases per task, whole words
    const uint64_t tasks = (n + SPAN - 1) / SPAN;
    std::vector<std::vector<ByteRun>> found(tasks);
    run_parallel(tasks, C.threads, [&](uint64_t k) {
        std::vector<ByteRun>& runs = found[k];
        const uint64_t q1 = std::min(n, (k + 1) * SPAN);
        for (uint64_t w = k * SPAN; w < q1; w += 16) {
            uint32_t word = 0;
            for (uint64_t q = w; q < std::min(w + 16, q1); q++) {
                const uint8_t c = code[R[q]];
                if (c < 4) word |= (uint32_t)c << (2 * (q - w));
                else if (!runs.empty() && runs.back().end == q && runs.back().byte == R[q]) runs.back().end++;
                else runs.push_back({q, q + 1, R[q]});
            }
            C.PW[w / 16] = word;
        }
    });
    for (const auto& part : found)                             // a run cut by a task edge is one run
        for (const ByteRun& r : part) {
            if (!C.PES.empty() && (uint64_t)(C.PES.back() + C.PEL.back()) == r.start && C.PEB.back() == r.byte) {
                C.PEL.back() += (int64_t)(r.end - r.start);
                continue;
            }
            C.PES.push_back((int64_t)r.start); C.PEL.push_back((int64_t)(r.end - r.start)); C.PEB.push_back(r.byte);
        }
    std::vector<int64_t> ends(C.PES.size());
    for (size_t r = 0; r < ends.size(); r++) ends[r] = C.PES[r] + C.PEL[r];
    C.PEIX.resize((n >> PV_EXC_BUCKET_BITS) + 2);
    for (uint64_t k = 0; k < C.PEIX.size(); k++)
        C.PEIX[k] = (uint32_t)(std::upper_bound(ends.begin(), ends.end(), (int64_t)(k << PV_EXC_BUCKET_BITS)) - ends.begin());
    std::vector<uint8_t>().swap(C.ref);
}

// The cohort's pooled arrays (layouts in include/panvram_amd.h), archive by archive in open order
void pool(pv_cohort& C) {
    const size_t n = C.A.size();
    const bool compact = C.form & PV_FORM_COMPACT_BLOCKS;
    std::vector<Placement> at(n + 1);
    for (size_t i = 0; i < n; i++) {
        const Archive& X = *C.A[i];
        Placement next = at[i];
        next.payload += X.payload_bytes;
        next.blocks += X.nb + 1;
        next.runs += X.low_s.size();
        next.contigs += X.rec.size();
        next.groups += (X.nb + PV_GROUP - 1) / PV_GROUP;
        at[i + 1] = next;
    }
    const Placement& total = at[n];
    C.P.assign(total.payload + 64, 0);                          // 64 zero bytes after the last payload
    if (compact) {
        const uint64_t groups = std::max<uint64_t>(total.groups, 1);
        C.BLEN.assign(total.blocks, 0); C.BCODE.assign(total.blocks, 0);
        C.GRP_OFF.assign(groups, 0); C.GRP_ST.assign(groups, 0); C.RUN0G.assign(groups, 0);
    } else {
        C.OFF.resize(total.blocks); C.ST.resize(total.blocks); C.RUN0.resize(total.blocks);
    }
    C.TAB.assign(n * pvc::GTAB_BYTES, 0);
    C.ASM.assign(n * 8, 0);
    C.LOW_S.resize(total.runs); C.LOW_L.resize(total.runs);
    for (auto* v : {&C.CTG_ASM, &C.CTG_LOCAL, &C.CTG_BOFF, &C.CTG_LEN}) v->resize(total.contigs);
    std::vector<std::vector<std::pair<int64_t, int64_t>>> exc(n);
    std::vector<std::string> refused(n);
    run_parallel(n, C.threads, [&](uint64_t i) {
        Archive& X = *C.A[i];
        const Placement& p = at[i];
        std::copy(X.payload.begin(), X.payload.end(), C.P.begin() + (ptrdiff_t)p.payload);
        const std::vector<uint32_t> run0 = first_runs(X);
        if (compact) {
            try { place_compact(X, run0, p, C, exc[i]); } catch (const FormatErr& e) { refused[i] = e.what(); }
        } else {
            std::copy(X.off.begin(), X.off.end(), C.OFF.begin() + (ptrdiff_t)p.blocks);
            std::copy(X.st.begin(), X.st.end(), C.ST.begin() + (ptrdiff_t)p.blocks);
            std::copy(run0.begin(), run0.end(), C.RUN0.begin() + (ptrdiff_t)p.blocks);
        }
        build_gtab(X, &C.TAB[i * pvc::GTAB_BYTES]);
        const int64_t rec[8] = {(int64_t)p.payload, (int64_t)p.blocks, (int64_t)X.nbases, (int64_t)p.runs,
                                (int64_t)X.low_s.size(), (int64_t)p.groups, 0, 0};
        std::copy(rec, rec + 8, C.ASM.begin() + (ptrdiff_t)(8 * i));
        std::copy(X.low_s.begin(), X.low_s.end(), C.LOW_S.begin() + (ptrdiff_t)p.runs);
        std::copy(X.low_l.begin(), X.low_l.end(), C.LOW_L.begin() + (ptrdiff_t)p.runs);
        for (size_t k = 0; k < X.rec.size(); k++) {
            const uint64_t row = p.contigs + k;
            C.CTG_ASM[row] = (int64_t)i; C.CTG_LOCAL[row] = (int64_t)k;
            C.CTG_BOFF[row] = (int64_t)X.rec[k].boff; C.CTG_LEN[row] = (int64_t)X.rec[k].len;
        }
        // the archive keeps its case runs (FASTA and case application read them); the rest now lives in the pool
        std::vector<uint8_t>().swap(X.payload); std::vector<uint32_t>().swap(X.off); std::vector<int64_t>().swap(X.st);
    });
    for (const std::string& r : refused)
        if (!r.empty()) throw FormatErr(r);
    for (const auto& part : exc)                               // in pooled block order: archive by archive
        for (const auto& e : part) { C.EXC_B.push_back(e.first); C.EXC_ST.push_back(e.second); }
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
        C->ref_path = reference; C->threads = threads > 0 ? threads : online_cpus(); C->form = form;
        C->ref = load_file(reference);
        C->ref_n = fasta_to_bases(C->ref.data(), C->ref.size(), reference);
        C->ref.resize(C->ref_n); C->ref.shrink_to_fit();
        pvs::sha256(C->ref.data(), C->ref_n, C->ref_sha);
        if (C->ref_n >= (1ull << 32)) throw FormatErr("reference of 2^32 bases or more: copy positions are 32-bit");
        C->A.resize((size_t)npaths);
        std::mutex mu; std::string first; bool first_is_format = true;
        run_parallel((uint64_t)npaths, C->threads, [&](uint64_t i) {
            try {
                const std::vector<uint8_t> f = load_file(paths[i]);
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
    const std::string h = to_hex(c->ref_sha, 32); memcpy(out_hex, h.c_str(), 65);
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
    run_parallel((X->nb + per - 1) / per, c->threads, [&](uint64_t g) {
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
        std::vector<uint8_t> b = load_file(path);
        const uint64_t n = fasta_to_bases(b.data(), b.size(), path);
        uint8_t s[32]; pvs::sha256(b.data(), n, s);
        const std::string h = to_hex(s, 32); memcpy(out_hex, h.c_str(), 65);
        return PV_OK;
    } catch (const FormatErr& e) { set_err(err, errcap, e.what()); return PV_EFORMAT; }
    catch (const std::exception& e) { set_err(err, errcap, e.what()); return PV_EARG; }
}

}  // extern "C"
