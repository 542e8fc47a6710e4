/* pv_oracle.c - CPU restatement of the reference's refrel3 v1 decoder. TEST INFRASTRUCTURE ONLY: the parity checker
 * for the HIP path and the timed CPU baseline in bench.py. Nothing in panvram_amd/ links, loads or calls it; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * Every function names the reference code it restates (paths under the reference repository). It keeps the
 * reference's formulation on purpose - a 4096-entry symbol lookup table per context built from the frequencies
 * (csrc/pv_v1.h:56-58), an op array filled by the block decoder and executed afterwards (csrc/refrel3.h:161-169,
 * csrc/pv_v1.h:65-72), a std::thread-style pool with an atomic work counter (csrc/pv_core.cpp:15-20) - so that it
 * checks the GPU kernels' different formulation (cumulative-count lookup, LDS replay) rather than restating it.
 *
 * Pinned by (tests/test_oracle.py): the per-block XXH3 of all six reference fixture archives (every block of
 * synth{A,B}.{q1k,q4k,q16k}.rr3), the base-stream XXH3 and the source-FASTA XXH3 in their headers, the reference
 * SHA-256 in their headers, the harness build of the reference's own decoder (oracle/_ref) where it builds, and
 * closed forms for the window transforms (reverse complement twice = identity, tokens of complements = 3 - token).
 */
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* zstd runtime (system libzstd.so.1) */
unsigned long long ZSTD_getFrameContentSize(const void* src, size_t srcSize);
size_t ZSTD_findFrameCompressedSize(const void* src, size_t srcSize);
size_t ZSTD_decompress(void* dst, size_t dstCapacity, const void* src, size_t compressedSize);

/* ------------------------------------------------------------------ constants (csrc/refrel3.h:24-43) */
enum { LL = 0, LITR = 4, LIT2 = 14, KIND = 31, DELTA = 47, REPK = 49, REPD = 50, DIRC = 51, SELFC = 52, LEN = 53, FLIPK = 59, FLIPD = 60, NCTX = 61 };
enum { CONT = 0, KDELTA = 1, REP = 2, ABS_ = 3, SELF = 4, FLIP = 5 };
#define AB 104
#define PB 12u
#define MM (1u << PB)
#define RL (1u << 16)
#define MINL 12u
#define MAXOPS 4096u
static const int ALPHA[NCTX] = {AB, AB, AB, AB, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6,
                                6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, 6, AB, AB, 3, AB, 2, AB, AB, AB, AB, AB, AB, AB, 4, AB};

typedef struct { uint16_t freq[NCTX][AB]; uint16_t cum[NCTX][AB + 1]; uint8_t sym[NCTX][MM]; } Tab;   /* csrc/refrel3.h:66 */
typedef struct { uint64_t src; uint32_t dst, len, kind; } Op;                                          /* csrc/refrel_format.h:34 */

typedef struct {
    uint32_t Q, flags; uint64_t nbases, nb, fasta_xxh, bases_xxh, payload_bytes;
    uint32_t nrec; char** hdr; uint64_t* rlen; uint64_t* rboff; uint32_t* lw;
    uint64_t nlow; uint64_t* low_s; uint64_t* low_l;
    uint64_t* hashes; Tab* T; uint32_t* off; int64_t* st; uint8_t* P;
} Arch;

static uint64_t rd64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }
static uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }

/* ------------------------------------------------------------------ reference FASTA -> bases (csrc/pv_v1.h:42-53) */
int64_t oracle_fasta_bases(uint8_t* b, uint64_t n) {
    if (!n || b[0] != '>') return -1;
    uint64_t i = 0, w = 0;
    while (i < n) {
        const uint8_t* e = (const uint8_t*)memchr(b + i, '\n', n - i);
        if (b[i] == '>') { if (!e) return -1; i = (uint64_t)(e - b) + 1; continue; }
        if (!e) return -1;
        for (uint64_t k = i; k < (uint64_t)(e - b); k++) { const uint8_t c = b[k]; b[w++] = (c >= 'a' && c <= 'z') ? (uint8_t)(c - 32) : c; }
        i = (uint64_t)(e - b) + 1;
    }
    return (int64_t)w;
}

/* ------------------------------------------------------------------ tables (csrc/pv_v1.h:56-58 build_tab) */
static void build_tab(Tab* T) {
    for (int c = 0; c < NCTX; c++) {
        uint32_t a = 0;
        for (int s = 0; s < AB; s++) { T->cum[c][s] = (uint16_t)a; for (uint32_t k = 0; k < T->freq[c][s]; k++) T->sym[c][a + k] = (uint8_t)s; a += T->freq[c][s]; }
        T->cum[c][AB] = (uint16_t)a;
    }
}

void oracle_close(Arch* X) {
    if (!X) return;
    for (uint32_t r = 0; r < X->nrec && X->hdr; r++) free(X->hdr[r]);
    free(X->hdr); free(X->rlen); free(X->rboff); free(X->lw); free(X->low_s); free(X->low_l); free(X->hashes);
    free(X->T); free(X->off); free(X->st); free(X->P); free(X);
}

/* ------------------------------------------------------------------ open (csrc/pv_v1.h:99-146 open_v1). The header XXH3
 * and the reference SHA-256 checks are left to the Python side of the tests (xxhash / hashlib): this function is the
 * decoder's reader, and returns a short reason code on refusal (0 = ok). */
int oracle_open(const uint8_t* a, uint64_t n, Arch** out) {
    *out = NULL;
    if (n < 138) return 1;
    if (memcmp(a, "RFRL3V1\0", 8)) return 2;
    if (rd32(a + 8) != 1) return 3;
    Arch* X = (Arch*)calloc(1, sizeof(Arch));
    X->Q = rd32(a + 12);
    if (!(X->Q == 1024 || X->Q == 2048 || X->Q == 4096 || X->Q == 16384)) { oracle_close(X); return 4; }
    X->flags = rd32(a + 16);
    if ((X->flags & ~1u) || rd32(a + 20)) { oracle_close(X); return 5; }
    X->nbases = rd64(a + 64); X->nb = rd64(a + 72); X->fasta_xxh = rd64(a + 80); X->bases_xxh = rd64(a + 88);
    const uint64_t mz = rd64(a + 96), mr = rd64(a + 104), hs = rd64(a + 112), pl = rd64(a + 120);
    const uint16_t nl = (uint16_t)(a[136] | a[137] << 8);
    const uint64_t pstart = 138ull + nl + mz + hs;
    if (mz > n || hs > n || pl > n || pstart > n || pstart + pl != n) { oracle_close(X); return 6; }
    if (X->nb != (X->nbases + X->Q - 1) / X->Q) { oracle_close(X); return 7; }
    if (hs != ((X->flags & 1) ? X->nb * 8 : 0)) { oracle_close(X); return 8; }
    const uint8_t* mzp = a + 138 + nl;
    if (mr > (1ull << 32) || ZSTD_getFrameContentSize(mzp, mz) != mr || ZSTD_findFrameCompressedSize(mzp, mz) != mz) { oracle_close(X); return 9; }
    uint8_t* M = (uint8_t*)malloc(mr ? mr : 1);
    if (ZSTD_decompress(M, mr, mzp, mz) != mr) { free(M); oracle_close(X); return 10; }
    uint64_t i = 0; int bad = 0;
#define NEED(k) ((i + (k) > mr) ? (bad = 1, 0) : 1)
    uint64_t v;
#define LEB(dst) do { uint64_t _v = 0; int _sh = 0; for (;;) { if (!NEED(1) || _sh > 63) { bad = 1; _v = 0; break; } const uint8_t _c = M[i++]; _v |= (uint64_t)(_c & 0x7F) << _sh; if (!(_c & 0x80)) break; _sh += 7; } (dst) = _v; } while (0)
    X->nrec = NEED(4) ? rd32(M + i) : 0; if (!bad) i += 4;
    if (X->nrec > mr) { free(M); oracle_close(X); return 11; }
    X->hdr = (char**)calloc(X->nrec + 1, sizeof(char*)); X->rlen = (uint64_t*)calloc(X->nrec + 1, 8);
    X->rboff = (uint64_t*)calloc(X->nrec + 1, 8); X->lw = (uint32_t*)calloc(X->nrec + 1, 4);
    uint64_t bo = 0;
    for (uint32_t r = 0; r < X->nrec && !bad; r++) {
        if (!NEED(4)) break;
        const uint32_t hl = rd32(M + i); i += 4;
        if (!NEED(hl)) break;
        X->hdr[r] = (char*)malloc(hl + 1); memcpy(X->hdr[r], M + i, hl); X->hdr[r][hl] = 0; i += hl;
        if (!NEED(12)) break;
        X->rlen[r] = rd64(M + i); i += 8; X->lw[r] = rd32(M + i); i += 4;
        if (!X->lw[r] && X->rlen[r]) bad = 1;
        X->rboff[r] = bo; bo += X->rlen[r];
    }
    if (bad || bo != X->nbases) { free(M); oracle_close(X); return 12; }
    if (!NEED(8)) { free(M); oracle_close(X); return 13; }
    X->nlow = rd64(M + i); i += 8;
    if (X->nlow > X->nbases) { free(M); oracle_close(X); return 13; }
    X->low_s = (uint64_t*)malloc((X->nlow + 1) * 8); X->low_l = (uint64_t*)malloc((X->nlow + 1) * 8);
    uint64_t last = 0;
    for (uint64_t k = 0; k < X->nlow && !bad; k++) {
        uint64_t g, l; LEB(g); LEB(l);
        if (last + g + l > X->nbases) { bad = 1; break; }
        X->low_s[k] = last + g; X->low_l[k] = l; last += g + l;
    }
    if (bad) { free(M); oracle_close(X); return 13; }
    X->T = (Tab*)calloc(1, sizeof(Tab));
    for (int c = 0; c < NCTX && !bad; c++) {
        uint64_t sum = 0;
        for (int s = 0; s < ALPHA[c]; s++) { LEB(v); if (v > MM) bad = 1; X->T->freq[c][s] = (uint16_t)v; sum += v; }
        if (sum && sum != MM) bad = 1;
    }
    if (bad) { free(M); oracle_close(X); return 14; }
    build_tab(X->T);
    if (pl >= (1ull << 32)) { free(M); oracle_close(X); return 15; }
    X->off = (uint32_t*)calloc(X->nb + 1, 4); X->st = (int64_t*)calloc(X->nb + 1, 8);
    uint64_t prevc = 0; uint32_t prevd = 0, acc = 0;
    for (uint64_t b = 0; b < X->nb && !bad; b++) {
        uint64_t len; LEB(len); if (bad || len > pl - acc) { bad = 1; break; }
        acc += (uint32_t)len; X->off[b + 1] = acc;
        LEB(v);
        const int64_t pred = b == 0 ? 0 : (int64_t)(prevd ? prevc - X->Q : prevc + X->Q);
        const uint64_t q = v >> 1;
        const uint64_t c = (uint64_t)(pred + ((int64_t)(q >> 1) ^ -(int64_t)(q & 1)));
        const uint32_t d = (uint32_t)(v & 1);
        X->st[b] = (int64_t)(c << 1) | (int64_t)d; prevc = c; prevd = d;
    }
    const int tail = (i != mr);
    free(M);
    if (bad || tail || acc != pl) { oracle_close(X); return 16; }
    if (X->flags & 1) { X->hashes = (uint64_t*)malloc(X->nb * 8 + 8); memcpy(X->hashes, a + 138 + nl + mz, X->nb * 8); }
    X->P = (uint8_t*)malloc(pl + 64); memcpy(X->P, a + pstart, pl); memset(X->P + pl, 0, 64); X->payload_bytes = pl;
    *out = X;
    return 0;
#undef NEED
#undef LEB
}

/* ------------------------------------------------------------------ rANS (csrc/refrel3.h:68-91) */
typedef struct { const uint8_t* p; const uint8_t* e; uint32_t x; int bad; } Dec;
static void dinit(Dec* d, const uint8_t* p, uint32_t n) {
    d->p = p; d->e = p + n; d->bad = 0; d->x = 0;
    if (n < 3) { d->bad = 1; return; }
    d->x = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16); d->p += 3;
}
static uint32_t dsym(Dec* d, const Tab* T, int c) {
    const uint32_t slot = d->x & (MM - 1), s = T->sym[c][slot], f = T->freq[c][s];
    if (!f) { d->bad = 1; return 0; }
    d->x = f * (d->x >> PB) + slot - T->cum[c][s];
    while (d->x < RL) { if (d->p >= d->e) { d->bad = 1; return s; } d->x = (d->x << 8) | *d->p++; }
    return s;
}
static uint64_t draw(Dec* d, uint32_t nb) {
    uint64_t v = 0; uint32_t sh = 0;
    while (nb) {
        const uint32_t k = nb > 16 ? 16 : nb, b = d->x & ((1u << k) - 1); d->x >>= k;
        while (d->x < RL) { if (d->p >= d->e) { d->bad = 1; return v; } d->x = (d->x << 8) | *d->p++; }
        v |= (uint64_t)b << sh; sh += k; nb -= k;
    }
    return v;
}
static uint64_t unbucket(uint32_t s, uint64_t extra) {          /* csrc/refrel3.h:55-59 */
    if (s < 16) return s;
    const uint32_t e = (s - 16) / 4 + 4, m = (s - 16) & 3;
    return (1ull << e) | ((uint64_t)m << (e - 2)) | extra;
}
static uint32_t nbits(uint32_t s) { return s < 16 ? 0 : (s - 16) / 4 + 2; }
static uint64_t dval(Dec* d, const Tab* T, int c) { const uint32_t s = dsym(d, T, c); return unbucket(s, draw(d, nbits(s))); }
static int llc(uint64_t ll) { return ll == 0 ? 0 : ll == 1 ? 1 : ll <= 8 ? 2 : 3; }            /* csrc/refrel3.h:61-63 */
static int kclass(int k) { return k < 0 ? 0 : k == CONT ? 1 : (k == KDELTA || k == REP || k == FLIP) ? 2 : 3; }
static int b2(uint8_t c) { switch (c) { case 'A': return 0; case 'C': return 1; case 'G': return 2; case 'T': return 3; case 'N': return 4; default: return 5; } }
static uint8_t comp(uint8_t c) { switch (c) { case 'A': return 'T'; case 'C': return 'G'; case 'G': return 'C'; case 'T': return 'A'; default: return c; } }

/* ------------------------------------------------------------------ diagonals (csrc/refrel3.h:94-109) */
typedef struct { uint64_t c; uint32_t dir; } Diag;
static int64_t dexp(Diag g, uint32_t o, uint64_t L) { return g.dir ? (int64_t)g.c - (int64_t)o - (int64_t)L + 1 : (int64_t)g.c + (int64_t)o; }
static int64_t dlocus(Diag g, uint32_t o) { return g.dir ? (int64_t)g.c - (int64_t)o : (int64_t)g.c + (int64_t)o; }
static Diag mkdiag(uint32_t dir, uint64_t p, uint32_t o, uint64_t L) {
    Diag g; g.dir = dir; g.c = dir ? (uint64_t)((int64_t)p + (int64_t)L - 1 + (int64_t)o) : (uint64_t)((int64_t)p - (int64_t)o); return g;
}
static void push(Diag* cache, int* nc, Diag g) {
    int j = 0; while (j < *nc && !(cache[j].c == g.c && cache[j].dir == g.dir)) j++;
    if (j == *nc) { if (*nc < 4) (*nc)++; j = *nc - 1; }
    for (; j > 0; j--) cache[j] = cache[j - 1];
    cache[0] = g;
}
static int refbase(const uint8_t* ref, uint64_t ref_n, Diag g, uint32_t o) {
    const int64_t q = g.dir ? (int64_t)g.c - (int64_t)o : (int64_t)g.c + (int64_t)o;
    if (q < 0 || (uint64_t)q >= ref_n) return 4;
    const uint8_t b = g.dir ? comp(ref[q]) : ref[q]; const int k = b2(b); return k < 4 ? k : 4;
}

/* ------------------------------------------------------------------ block grammar -> ops + literals
 * (csrc/refrel3.h:114-160 r3_decode_stream with the array sink of :161-169). Returns the op count or -1. */
static int decode_ops(const uint8_t* src, uint32_t n, const Tab* T, const uint8_t* ref, uint64_t ref_n, uint32_t blen, Diag start,
                      Op* ops, uint32_t maxops, uint8_t* lit, uint32_t litcap) {
    Dec d; dinit(&d, src, n); if (d.bad) return -1;
    Diag cache[4]; int nc = 1; cache[0] = start; int prevk = -1; uint32_t o = 0, k = 0, li = 0;
    static const uint8_t B[6] = {'A', 'C', 'G', 'T', 'N', 0};
#define OP(KIND_, SRC_, DST_, LEN_) do { if (k >= maxops) return -1; ops[k].kind = (KIND_); ops[k].src = (SRC_); ops[k].dst = (DST_); ops[k].len = (LEN_); k++; } while (0)
    while (o < blen) {
        const uint64_t ll = dval(&d, T, LL + kclass(prevk));
        if (d.bad || ll > blen - o) return -1;
        if (ll) {
            uint32_t p1 = 16, p2 = 16;
            for (uint32_t j = 0; j < ll; j++) {
                int c;
                if (ll <= 8) c = LITR + refbase(ref, ref_n, cache[0], o + j) * 2 + (j == 0 ? 1 : 0);
                else c = LIT2 + (p1 == 16 ? 16 : (int)(p2 == 16 ? p1 : p2 * 4 + p1) % 16);
                const uint32_t s = dsym(&d, T, c);
                if (li + j >= litcap) return -1;
                lit[li + j] = s < 5 ? B[s] : (uint8_t)draw(&d, 8);
                p2 = p1; p1 = s < 4 ? s : 0;
            }
            OP(0, li, o, (uint32_t)ll);
            li += (uint32_t)ll; o += (uint32_t)ll;
        }
        if (o == blen) break;
        const int kind = (int)dsym(&d, T, KIND + llc(ll) * 4 + kclass(prevk));
        uint64_t p = 0; uint32_t dir = 0; int ki = 0; int64_t dd = 0; uint64_t dist = 0;
        if (kind == CONT || kind == KDELTA) {
            if (kind == KDELTA) { const uint64_t z = dval(&d, T, DELTA + (ll == 0 ? 0 : 1)); dd = (int64_t)(z >> 1) ^ -(int64_t)(z & 1); }
        } else if (kind == REP) {
            ki = 1 + (int)dsym(&d, T, REPK); const uint64_t z = dval(&d, T, REPD); dd = (int64_t)(z >> 1) ^ -(int64_t)(z & 1);
            if (ki >= nc) return -1;
        } else if (kind == ABS_) { dir = dsym(&d, T, DIRC); p = draw(&d, 32); }
        else if (kind == SELF) dist = dval(&d, T, SELFC);
        else if (kind == FLIP) {
            ki = (int)dsym(&d, T, FLIPK); const uint64_t z = dval(&d, T, FLIPD); dd = (int64_t)(z >> 1) ^ -(int64_t)(z & 1);
            if (ki >= nc) return -1;
        } else return -1;
        const uint64_t L = dval(&d, T, LEN + kind) + MINL;
        if (d.bad || L > blen - o) return -1;
        uint32_t okind; uint64_t osrc;
        if (kind == SELF) { if (dist == 0 || dist > o) return -1; okind = 2; osrc = o - dist; }
        else {
            if (kind == FLIP) { const Diag g = cache[ki]; dir = g.dir ^ 1; const int64_t e = dlocus(g, o) + dd; if (e < 0) return -1; p = (uint64_t)e; }
            else if (kind != ABS_) { const Diag g = cache[kind == REP ? ki : 0]; dir = g.dir; const int64_t e = dexp(g, o, L) + dd; if (e < 0) return -1; p = (uint64_t)e; }
            if (p > ref_n || L > ref_n - p) return -1;
            okind = dir ? 3 : 1; osrc = p; push(cache, &nc, mkdiag(dir, p, o, L));
        }
        OP(okind, osrc, o, (uint32_t)L);
        o += (uint32_t)L; prevk = kind;
    }
    if (d.bad || d.x != RL || d.p != d.e) return -1;
    return (int)k;
#undef OP
}

/* ------------------------------------------------------------------ op execution (csrc/pv_v1.h:65-72 exec_ops) */
static void exec_ops(const Op* ops, int n, const uint8_t* lit, const uint8_t* ref, uint8_t* out) {
    for (int k = 0; k < n; k++) {
        const Op* q = &ops[k];
        if (q->kind == 0) memcpy(out + q->dst, lit + q->src, q->len);
        else if (q->kind == 1) memcpy(out + q->dst, ref + q->src, q->len);
        else if (q->kind == 2) {
            const uint32_t dist = q->dst - (uint32_t)q->src;
            if (dist >= q->len) memcpy(out + q->dst, out + q->src, q->len);
            else for (uint32_t j = 0; j < q->len; j++) out[q->dst + j] = out[q->src + j];
        } else { const uint64_t r = q->src + q->len - 1; for (uint32_t j = 0; j < q->len; j++) out[q->dst + j] = comp(ref[r - j]); }
    }
}

typedef struct { Op* ops; uint8_t* lit; uint8_t* blk; } Scratch;
static int scratch_init(Scratch* S, uint32_t Q) {
    S->ops = (Op*)malloc(MAXOPS * sizeof(Op)); S->lit = (uint8_t*)malloc(Q); S->blk = (uint8_t*)malloc(Q);
    return S->ops && S->lit && S->blk;
}
static void scratch_free(Scratch* S) { free(S->ops); free(S->lit); free(S->blk); }

/* block b (upper case) into out: 0 ok, 1 decode failure (csrc/pv_v1.h:150-158 decode_block, verify left to Python) */
int oracle_decode_block_s(const Arch* X, const uint8_t* ref, uint64_t ref_n, uint64_t b, uint8_t* out, Scratch* S) {
    if (b >= X->nb) return 1;
    const uint32_t blen = (uint32_t)((X->nbases - b * X->Q) < X->Q ? X->nbases - b * X->Q : X->Q);
    const uint32_t o = X->off[b], l = X->off[b + 1] - X->off[b];
    Diag g; g.c = (uint64_t)(X->st[b] >> 1); g.dir = (uint32_t)(X->st[b] & 1);
    const int k = decode_ops(X->P + o, l, X->T, ref, ref_n, blen, g, S->ops, MAXOPS, S->lit, X->Q);
    if (k < 0) return 1;
    exec_ops(S->ops, k, S->lit, ref, out);
    return 0;
}
int oracle_decode_block(const Arch* X, const uint8_t* ref, uint64_t ref_n, uint64_t b, uint8_t* out) {
    Scratch S; if (!scratch_init(&S, X->Q)) return 1;
    const int e = oracle_decode_block_s(X, ref, ref_n, b, out, &S);
    scratch_free(&S); return e;
}

/* bases [s, s+W) with lower-case runs applied if asked (csrc/pv_v1.h:160-174 first_run + window_cpu) */
static int window_s(const Arch* X, const uint8_t* ref, uint64_t ref_n, uint64_t s, uint64_t W, uint8_t* out, Scratch* S, int apply_case) {
    if (!W) return 0;
    for (uint64_t b = s / X->Q; b <= (s + W - 1) / X->Q; b++) {
        if (oracle_decode_block_s(X, ref, ref_n, b, S->blk, S)) return 1;
        const uint64_t bs = b * X->Q, x0 = s > bs ? s : bs, x1 = (s + W) < (bs + X->Q) ? (s + W) : (bs + X->Q);
        memcpy(out + (x0 - s), S->blk + (x0 - bs), x1 - x0);
    }
    if (apply_case) {
        uint64_t lo = 0, hi = X->nlow;
        while (lo < hi) { const uint64_t m = (lo + hi) / 2; if (X->low_s[m] + X->low_l[m] <= s) lo = m + 1; else hi = m; }
        for (uint64_t r = lo; r < X->nlow && X->low_s[r] < s + W; r++) {
            const uint64_t x0 = s > X->low_s[r] ? s : X->low_s[r], e = X->low_s[r] + X->low_l[r], x1 = (s + W) < e ? (s + W) : e;
            for (uint64_t x = x0; x < x1; x++) out[x - s] |= 0x20;
        }
    }
    return 0;
}

/* output transforms (csrc/pv_v1.h:74-76, applied as csrc/pv_core.cpp:129-132) */
static uint8_t comp_case(uint8_t c) {
    switch (c) { case 'A': return 'T'; case 'C': return 'G'; case 'G': return 'C'; case 'T': return 'A';
                 case 'a': return 't'; case 'c': return 'g'; case 'g': return 'c'; case 't': return 'a'; default: return c; }
}
static uint8_t token(uint8_t c) { switch (c | 0x20) { case 'a': return 0; case 'c': return 1; case 'g': return 2; case 't': return 3; default: return 4; } }

/* ------------------------------------------------------------------ windows over many archives, thread pool
 * (csrc/pv_core.cpp:15-20 parallel, :116-136 Core::windows): windows dealt in contiguous chunks of
 * ceil(n / (4T)), one scratch per chunk, first error wins. Returns 0, 1 (decode failure) or 3 (window outside). */
typedef struct {
    Arch* const* A; int64_t nA; const uint8_t* ref; uint64_t ref_n;
    const int64_t* asmv; const int64_t* start; int64_t n; int64_t W; const uint8_t* rc; int tokens, apply_case;
    uint8_t* out; uint64_t chunk, nchunks; volatile int64_t next; volatile int err;
} Job;

static void* worker(void* arg) {
    Job* J = (Job*)arg;
    for (;;) {
        const uint64_t c = (uint64_t)__atomic_fetch_add(&J->next, 1, __ATOMIC_RELAXED);
        if (c >= J->nchunks) break;
        Scratch S; if (!scratch_init(&S, J->A[0]->Q)) { __atomic_store_n(&J->err, 1, __ATOMIC_RELAXED); break; }
        const uint64_t w1 = (c + 1) * J->chunk < (uint64_t)J->n ? (c + 1) * J->chunk : (uint64_t)J->n;
        for (uint64_t w = c * J->chunk; w < w1 && !__atomic_load_n(&J->err, __ATOMIC_RELAXED); w++) {
            uint8_t* o = J->out + w * (uint64_t)J->W;
            if (window_s(J->A[J->asmv[w]], J->ref, J->ref_n, (uint64_t)J->start[w], (uint64_t)J->W, o, &S, J->apply_case && !J->tokens)) {
                int z = 0; __atomic_compare_exchange_n(&J->err, &z, 1, 0, __ATOMIC_RELAXED, __ATOMIC_RELAXED); break;
            }
            if (J->rc && J->rc[w]) {
                for (int64_t i = 0, j = J->W - 1; i < j; i++, j--) { const uint8_t t = comp_case(o[i]); o[i] = comp_case(o[j]); o[j] = t; }
                if (J->W & 1) o[J->W / 2] = comp_case(o[J->W / 2]);
            }
            if (J->tokens) for (int64_t i = 0; i < J->W; i++) o[i] = token(o[i]);
        }
        scratch_free(&S);
    }
    return NULL;
}

int oracle_windows(Arch* const* A, int64_t nA, const uint8_t* ref, uint64_t ref_n, const int64_t* asmv, const int64_t* start, int64_t n,
                   int64_t W, const uint8_t* rc, int tokens, int apply_case, int threads, uint8_t* out) {
    if (W < 0) return 2;
    for (int64_t w = 0; w < n; w++) {
        if (asmv[w] < 0 || asmv[w] >= nA) return 3;
        if (start[w] < 0 || (uint64_t)start[w] + (uint64_t)W > A[asmv[w]]->nbases) return 3;
    }
    if (n == 0) return 0;
    Job J; memset(&J, 0, sizeof J);
    J.A = A; J.nA = nA; J.ref = ref; J.ref_n = ref_n; J.asmv = asmv; J.start = start; J.n = n; J.W = W; J.rc = rc;
    J.tokens = tokens; J.apply_case = apply_case; J.out = out;
    const uint64_t T = threads > 0 ? (uint64_t)threads : 1;
    J.chunk = ((uint64_t)n + T * 4 - 1) / (T * 4); if (!J.chunk) J.chunk = 1;
    J.nchunks = ((uint64_t)n + J.chunk - 1) / J.chunk;
    const uint64_t nt = T < J.nchunks ? T : J.nchunks;
    pthread_t th[256]; const uint64_t m = nt < 256 ? nt : 256;
    for (uint64_t t = 0; t < m; t++) pthread_create(&th[t], NULL, worker, &J);
    for (uint64_t t = 0; t < m; t++) pthread_join(th[t], NULL);
    return J.err;
}

/* ------------------------------------------------------------------ accessors for the ctypes side */
uint32_t oracle_Q(const Arch* X) { return X->Q; }
uint64_t oracle_nbases(const Arch* X) { return X->nbases; }
uint64_t oracle_nblocks(const Arch* X) { return X->nb; }
uint64_t oracle_fasta_xxh(const Arch* X) { return X->fasta_xxh; }
uint64_t oracle_bases_xxh(const Arch* X) { return X->bases_xxh; }
int oracle_has_hashes(const Arch* X) { return X->hashes != NULL; }
uint64_t oracle_block_hash(const Arch* X, uint64_t b) { return X->hashes && b < X->nb ? X->hashes[b] : 0; }
uint32_t oracle_nrec(const Arch* X) { return X->nrec; }
const char* oracle_rec_hdr(const Arch* X, uint32_t r) { return r < X->nrec ? X->hdr[r] : NULL; }
uint64_t oracle_rec_len(const Arch* X, uint32_t r) { return r < X->nrec ? X->rlen[r] : 0; }
uint64_t oracle_rec_boff(const Arch* X, uint32_t r) { return r < X->nrec ? X->rboff[r] : 0; }
uint32_t oracle_rec_lw(const Arch* X, uint32_t r) { return r < X->nrec ? X->lw[r] : 0; }
uint64_t oracle_nlow(const Arch* X) { return X->nlow; }
uint64_t oracle_payload_len(const Arch* X, uint64_t b) { return b < X->nb ? X->off[b + 1] - X->off[b] : 0; }
uint64_t oracle_payload_off(const Arch* X, uint64_t b) { return b <= X->nb ? X->off[b] : 0; }
uint64_t oracle_payload_bytes(const Arch* X) { return X->payload_bytes; }
int64_t oracle_block_state(const Arch* X, uint64_t b) { return b <= X->nb ? X->st[b] : 0; }

/* full stream, upper case then case runs (csrc/pv_core.cpp:144-149): 0 ok, 1 decode failure */
int oracle_full(const Arch* X, const uint8_t* ref, uint64_t ref_n, uint8_t* out, int apply_case) {
    Scratch S; if (!scratch_init(&S, X->Q)) return 1;
    for (uint64_t b = 0; b < X->nb; b++) {
        const uint64_t bs = b * X->Q, len = (X->nbases - bs) < X->Q ? X->nbases - bs : X->Q;
        if (oracle_decode_block_s(X, ref, ref_n, b, S.blk, &S)) { scratch_free(&S); return 1; }
        memcpy(out + bs, S.blk, len);
    }
    scratch_free(&S);
    if (apply_case) for (uint64_t r = 0; r < X->nlow; r++) for (uint64_t x = X->low_s[r]; x < X->low_s[r] + X->low_l[r]; x++) out[x] |= 0x20;
    return 0;
}

/* bytes of block b produced by reference copies (ops of kind 1 and 3): the reference bytes a decoder must read for it;
 * -1 on a decode failure */
int64_t oracle_block_refbytes(const Arch* X, const uint8_t* ref, uint64_t ref_n, uint64_t b) {
    if (b >= X->nb) return -1;
    Scratch S; if (!scratch_init(&S, X->Q)) return -1;
    const uint32_t blen = (uint32_t)((X->nbases - b * X->Q) < X->Q ? X->nbases - b * X->Q : X->Q);
    Diag g; g.c = (uint64_t)(X->st[b] >> 1); g.dir = (uint32_t)(X->st[b] & 1);
    const int k = decode_ops(X->P + X->off[b], X->off[b + 1] - X->off[b], X->T, ref, ref_n, blen, g, S.ops, MAXOPS, S.lit, X->Q);
    int64_t t = k < 0 ? -1 : 0;
    for (int i = 0; i < k; i++) if (S.ops[i].kind == 1 || S.ops[i].kind == 3) t += S.ops[i].len;
    scratch_free(&S);
    return t;
}
