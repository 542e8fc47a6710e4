// ref_harness.cpp - a thin C entry layer over the REFERENCE's own CPU decoder, compiled from the reference sources
// where they lie (-I <reference>/csrc; nothing copied): reference loading (csrc/pv_v1.h:42-53 fasta_bases_inplace,
// csrc/rr_sha256.h), open with checks (csrc/pv_v1.h:99-146 open_v1), and windows (csrc/pv_v1.h:164-174 window_cpu,
// csrc/pv_v1.h:74-76 comp_case / token). Test infrastructure only (oracle/_ref); the window loop below restates
// csrc/pv_core.cpp:116-136 (Core::windows), whose file cannot be compiled without torch and pybind11.
#include "pv_v1.h"
#include <atomic>
#include <mutex>
#include <thread>

namespace {
struct Ref {
    std::vector<uint8_t> R; uint64_t n = 0; uint8_t sha[32];
    std::vector<std::unique_ptr<pv::Archive>> A;
};
void seterr(char* e, size_t cap, const std::string& m) { if (e && cap) { snprintf(e, cap, "%s", m.c_str()); } }
}

extern "C" {

// archives opened in parallel (as csrc/pv_core.cpp:43-47 does), `threads` <= 0: all cores
void* ref_open(const char* reference, const char* const* paths, int n, int threads, char* err, size_t cap) {
    try {
        std::unique_ptr<Ref> h(new Ref());
        h->R = pv::slurp(reference);
        h->n = pv::fasta_bases_inplace(h->R.data(), h->R.size(), reference);
        rr_sha256(h->R.data(), h->n, h->sha);
        h->A.resize(n);
        std::atomic<int> next{0}; std::mutex mu; std::string first; std::vector<std::thread> th;
        const int T = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
        for (int t = 0; t < std::min(T, std::max(n, 1)); t++) th.emplace_back([&] {
            for (;;) {
                const int i = next.fetch_add(1); if (i >= n) break;
                try {
                    const std::vector<uint8_t> f = pv::slurp(paths[i]);
                    std::unique_ptr<pv::Archive> X(new pv::Archive());
                    pv::open_v1(f, paths[i], h->sha, h->n, *X);
                    h->A[i] = std::move(X);
                } catch (const std::exception& e) { std::lock_guard<std::mutex> g(mu); if (first.empty()) first = e.what(); }
            }
        });
        for (auto& x : th) x.join();
        if (!first.empty()) { seterr(err, cap, first); return nullptr; }
        return h.release();
    } catch (const std::exception& e) { seterr(err, cap, e.what()); return nullptr; }
}

void ref_close(void* p) { delete (Ref*)p; }

// 0 ok, 1 decode failure, 2 block XXH3 mismatch (verify), 3 window outside an assembly
int ref_windows(void* p, const int64_t* asmv, const int64_t* start, int64_t n, int64_t W, const uint8_t* rc, int tokens,
                int apply_case, int verify, int threads, uint8_t* out) {
    Ref* h = (Ref*)p;
    for (int64_t w = 0; w < n; w++) {
        if (asmv[w] < 0 || asmv[w] >= (int64_t)h->A.size()) return 3;
        if (start[w] < 0 || (uint64_t)start[w] + (uint64_t)W > h->A[asmv[w]]->nbases) return 3;
    }
    if (!n) return 0;
    const uint64_t T = (uint64_t)std::max(1, threads);
    const uint64_t chunk = std::max<uint64_t>(1, ((uint64_t)n + T * 4 - 1) / (T * 4)), nchunks = ((uint64_t)n + chunk - 1) / chunk;
    std::atomic<uint64_t> next{0}; std::atomic<int> e{0}; std::vector<std::thread> th;
    const uint32_t Q = h->A[0]->Q;
    for (uint64_t t = 0; t < std::min(T, nchunks); t++) th.emplace_back([&] {
        for (;;) {
            const uint64_t c = next.fetch_add(1); if (c >= nchunks) break;
            pv::Scratch S(Q);
            for (uint64_t w = c * chunk; w < std::min<uint64_t>((uint64_t)n, (c + 1) * chunk) && !e; w++) {
                uint8_t* o = out + w * (uint64_t)W;
                const int r = pv::window_cpu(*h->A[asmv[w]], h->R.data(), h->n, (uint64_t)start[w], (uint64_t)W, o, S, apply_case && !tokens, verify != 0);
                if (r) { int z = 0; e.compare_exchange_strong(z, r); break; }
                if (rc && rc[w]) {
                    for (int64_t i = 0, j = W - 1; i < j; i++, j--) { const uint8_t t2 = pv::comp_case(o[i]); o[i] = pv::comp_case(o[j]); o[j] = t2; }
                    if (W & 1) o[W / 2] = pv::comp_case(o[W / 2]);
                }
                if (tokens) for (int64_t i = 0; i < W; i++) o[i] = pv::token(o[i]);
            }
        }
    });
    for (auto& x : th) x.join();
    return e;
}

// one block, upper case (csrc/pv_v1.h:150-158): 0 ok, 1 decode failure, 2 hash mismatch
int ref_block(void* p, int64_t a, uint64_t b, int verify, uint8_t* out) {
    Ref* h = (Ref*)p; pv::Scratch S(h->A[a]->Q);
    return pv::decode_block(*h->A[a], h->R.data(), h->n, b, out, S, verify != 0);
}

// bytes of block b of archive a produced by reference copies (kinds 1 and 3) - the reference's decoder
// (csrc/refrel3.h:164-169 r3_decode_block) run into an op array; -1 on a decode failure
int64_t ref_block_refbytes(void* p, int64_t a, uint64_t b) {
    Ref* h = (Ref*)p; const pv::Archive& X = *h->A[a]; pv::Scratch S(X.Q);
    const uint32_t blen = (uint32_t)std::min<uint64_t>(X.Q, X.nbases - b * X.Q);
    uint32_t o, l; R3Diag g; X.locate(b, &o, &l, &g);
    const int k = r3_decode_block(X.P + o, l, X.T, h->R.data(), h->n, blen, g, S.ops.data(), (uint32_t)S.ops.size(), S.lit.data(), (uint32_t)S.lit.size());
    if (k < 0) return -1;
    int64_t t = 0;
    for (int i = 0; i < k; i++) if (S.ops[i].kind == 1 || S.ops[i].kind == 3) t += S.ops[i].len;
    return t;
}

uint64_t ref_nbases(void* p, int64_t a) { return ((Ref*)p)->A[a]->nbases; }

}  // extern "C"
