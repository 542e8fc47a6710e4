/* panvram_amd.h - C ABI of the MI355X refrel3 v1 decode path (libpanvram_amd.so).
 *
 * Plain C types only (pointers, sizes, integers); no torch types, no C++ exceptions across the boundary. Every entry
 * point returns a pv_status (0 = success) and, where it can fail for a reason worth reporting, writes a NUL-terminated
 * message into a caller buffer (err, errcap). Host arrays returned by pointer are owned by the cohort handle and stay
 * valid until pv_cohort_release_array() / pv_cohort_close().
 *
 * The reference binds the same path through pybind11 (panvram._C, reference csrc/pv_core.cpp:195-220); each
 * declaration below names the reference interface it replaces; panvram_amd/_native.py binds them with ctypes.
 */
#ifndef PANVRAM_AMD_H
#define PANVRAM_AMD_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PV_ABI_VERSION 8

/* status codes */
#define PV_OK 0
#define PV_EFORMAT 1   /* refused archive / reference / decode of a corrupt block -> panvram.FormatError (ValueError) */
#define PV_EARG 2      /* invalid argument (bad Q, W, shapes, index) -> RuntimeError / IndexError on the Python side */
#define PV_EHIP 3      /* HIP runtime error (launch, attribute query) -> RuntimeError */
#define PV_ENOMEM 4    /* host allocation failed */

/* device status word bits written by the decode kernels (reference csrc/pv_cuda.cu:37, cohort.py:171-173) */
#define PV_ST_DECODE 1   /* a covering block failed to decode (corrupt archive) */
#define PV_ST_HASH 2     /* a block's XXH3 differs from the stored one (only with verify) */
#define PV_ST_WAIT 4     /* a bounded wait expired: sample's caller-stream wait for a ring stream (60 s), or a heavy list entry left undone */
#define PV_ST_RANGE 8    /* window outside its assembly (assembly index or [start, start+W) out of range) */

typedef struct pv_cohort pv_cohort; /* opaque host handle: reference, archives, pooled arrays */

/* ABI version of the loaded library (PV_ABI_VERSION it was built with). No reference counterpart. */
int32_t pv_abi_version(void);

/* Resident forms (pv_cohort_open's `form` bits). Replace Core's packed_reference / compact_blocks options (reference
 * csrc/pv_core.cpp:52-63,92-111, csrc/pv_compact.h): the same windows from fewer resident bytes.
 *  PV_FORM_PACKED_REF      the reference as 2 bits per base (PW) + runs of other bytes (PES, PEL, PEB) + a bucket
 *                          index of those runs (PEIX, one entry per 2^PV_EXC_BUCKET_BITS bases); no REF array
 *  PV_FORM_COMPACT_BLOCKS  the block table as groups of PV_GROUP blocks (GRP_OFF, GRP_ST, RUN0G) + a u16 payload
 *                          length and an i16 start code per block (BLEN, BCODE) + exceptions (EXC_B, EXC_ST); no OFF,
 *                          ST, RUN0 arrays. Refused ("... block payload over 65535 B ...") for larger block payloads. */
#define PV_FORM_PACKED_REF 1
#define PV_FORM_COMPACT_BLOCKS 2
#define PV_GROUP 32
#define PV_CODE_EXC (-32768)
#define PV_EXC_BUCKET_BITS 16

/* Open the reference FASTA and every archive with all checks of FORMAT.md section 5, pool their arrays.
 * Replaces pv::Core::Core (reference csrc/pv_core.cpp:32-50, with open_v1 csrc/pv_v1.h:99-146 and pool
 * csrc/pv_core.cpp:65-90). threads <= 0: all host cores. form: PV_FORM_* bits (0: the plain arrays). Errors:
 * PV_EFORMAT with "<path>: refused: <why>", "... wrong reference", "... block size ..." messages as the reference
 * words them; PV_EARG for unknown form bits. */
int32_t pv_cohort_open(const char* reference, const char* const* paths, int32_t npaths, int32_t threads, int32_t form,
                       pv_cohort** out, char* err, size_t errcap);
void pv_cohort_close(pv_cohort* c);

/* Scalars of the cohort. Replace Core.Q / .n / .ref_bases / .ref_sha256 (reference csrc/pv_core.cpp:205-210). */
int32_t pv_cohort_block_size(const pv_cohort* c);
int64_t pv_cohort_assemblies(const pv_cohort* c);
uint64_t pv_cohort_ref_bases(const pv_cohort* c);
void pv_cohort_ref_sha256(const pv_cohort* c, char out_hex[65]);
/* The form bits the cohort was opened with, and the lengths of its exception tables (reference runs of non-ACGT
 * bytes; blocks whose start needs the exception table). Replace Core.packed_reference / .compact_blocks and the
 * pne / nexc scalars of the reference's windows_cuda2 call (reference panvram/cohort.py:147-152). */
int32_t pv_cohort_form(const pv_cohort* c);
int64_t pv_cohort_ref_exceptions(const pv_cohort* c);
int64_t pv_cohort_block_exceptions(const pv_cohort* c);

/* Pooled host arrays, by id (the device copies are made once by the caller). Replaces Core.pools()
 * (reference csrc/pv_core.cpp:177-182). Layouts:
 *  P       u8 [sum payload + 64]     payload bytes, archives concatenated (+64 zero bytes)
 *  OFF     u32[sum (blocks+1)]       payload offset of block b relative to its archive's payload (b = blocks: size)
 *  ST      i64[sum (blocks+1)]       block start diagonal, (c << 1) | strand
 *  RUN0    u32[sum (blocks+1)]       first lower-case run (index within the archive) ending after b*Q
 *  TAB     u8 [A * 10240]            GPU model tables (cumulative frequencies per context, literal pairs, bucket entries; pv_codec.h)
 *  ASM     i64[A * 8]                per archive: pay_base, blk_base, bases, low_base, low_cnt, first group, 0, 0
 *  LOW_S   i64[sum runs]             lower-case run starts (per archive, sorted, disjoint)
 *  LOW_L   i64[sum runs]             lower-case run lengths
 *  REF     u8 [ref bases]            the decoded reference, upper case (empty with PV_FORM_PACKED_REF)
 *  CTG_ASM, CTG_LOCAL, CTG_BOFF, CTG_LEN   i64[sum contigs]   contig tables, cohort order
 * PV_FORM_PACKED_REF:
 *  PW      u32[ref bases / 16 + 1]   base q in bits 2 (q % 16) of word q / 16: A 0, C 1, G 2, T 3 (other bytes: 0)
 *  PES, PEL i64[runs]                maximal runs of one byte other than A/C/G/T: start, length (sorted, disjoint)
 *  PEB     u8 [runs]                 the run's byte
 *  PEIX    u32[ref bases / 2^16 + 2] for bucket k: the first run ending after base k * 2^16
 * PV_FORM_COMPACT_BLOCKS (the OFF / ST / RUN0 entries of block b of an archive then come from):
 *  GRP_OFF i64[sum groups]           per group of PV_GROUP blocks: OFF of its first block
 *  GRP_ST  i64[sum groups]           ST of its first block
 *  RUN0G   u32[sum groups]           RUN0 of its first block
 *  BLEN    u16[sum (blocks+1)]       payload length of the block
 *  BCODE   i16[sum (blocks+1)]       2 (c - predicted c) + strand, predicted c = previous c + Q (strand 0) or - Q;
 *                                    PV_CODE_EXC: ST is in the exception table; 0 for a group's first block
 *  EXC_B, EXC_ST i64[exceptions]     pooled block index (ASM blk_base + b), its ST; sorted by block index
 *  ASM[5] of each archive holds its first group's index. */
enum pv_array_id {
    PV_ARR_P = 0, PV_ARR_OFF, PV_ARR_ST, PV_ARR_RUN0, PV_ARR_TAB, PV_ARR_ASM, PV_ARR_LOW_S, PV_ARR_LOW_L, PV_ARR_REF,
    PV_ARR_CTG_ASM, PV_ARR_CTG_LOCAL, PV_ARR_CTG_BOFF, PV_ARR_CTG_LEN,
    PV_ARR_PW, PV_ARR_PES, PV_ARR_PEL, PV_ARR_PEB, PV_ARR_PEIX,
    PV_ARR_GRP_OFF, PV_ARR_GRP_ST, PV_ARR_RUN0G, PV_ARR_BLEN, PV_ARR_BCODE, PV_ARR_EXC_B, PV_ARR_EXC_ST, PV_ARR_COUNT
};
int32_t pv_cohort_array(const pv_cohort* c, int32_t id, const void** ptr, uint64_t* nbytes);
/* Free a pooled host array once its device copy exists (no reference counterpart: the reference keeps its CPU pools
 * for the CPU decoder, which this build keeps out of the product). */
int32_t pv_cohort_release_array(pv_cohort* c, int32_t id);

/* Per-assembly description. Replaces Core.info / Core.contigs (reference csrc/pv_core.cpp:160-163). */
typedef struct pv_asm_info {
    uint32_t Q, flags;
    uint64_t bases, blocks, file_bytes, payload_bytes, contigs, lower_case_runs;
    uint64_t fasta_xxh3, bases_xxh3;
    int32_t block_hashes;
    char path[1024];
    char reference_name[512];
} pv_asm_info;
int32_t pv_asm_info_get(const pv_cohort* c, int64_t a, pv_asm_info* out);
int32_t pv_asm_contig(const pv_cohort* c, int64_t a, int64_t k, const char** name, const char** header,
                      uint64_t* length, uint64_t* offset, uint32_t* line_width);

/* XXH3 of the FASTA file rebuilt from an assembly's decoded base stream (case applied) and its record layout,
 * streamed. Replaces Core::fasta_xxh3 (reference csrc/pv_core.cpp:167-176). */
int32_t pv_fasta_xxh3(const pv_cohort* c, int64_t a, const uint8_t* bases, uint64_t n, uint64_t* hash,
                      char* err, size_t errcap);
/* Size of the rebuilt FASTA, and the rebuild itself into out (capacity cap). Replaces the layout part of
 * Core::fasta (reference csrc/pv_core.cpp:138-159). */
uint64_t pv_fasta_size(const pv_cohort* c, int64_t a);
int32_t pv_fasta_build(const pv_cohort* c, int64_t a, const uint8_t* bases, uint64_t n, uint8_t* out, uint64_t cap,
                       char* err, size_t errcap);
/* Per-block XXH3 of an upper-case decoded stream against the archive's hash section; first_bad = -1 when all
 * agree (or the archive has no hashes). Replaces the verify step of pv::decode_block (reference csrc/pv_v1.h:156). */
int32_t pv_verify_blocks(const pv_cohort* c, int64_t a, const uint8_t* upper, uint64_t n, int64_t* first_bad);
/* Apply an assembly's lower-case runs in place to bases [s, s+n) of its stream (reference csrc/pv_v1.h:171-172). */
int32_t pv_apply_case(const pv_cohort* c, int64_t a, uint64_t s, uint8_t* bases, uint64_t n);
/* SHA-256 of a FASTA file's bases (upper case, no headers / line ends). Replaces _C.sha256_file_bases
 * (reference csrc/pv_core.cpp:211-212). */
int32_t pv_sha256_file_bases(const char* path, char out_hex[65], char* err, size_t errcap);

/* XXH3_64bits (seed 0) of a host buffer, and of the concatenation of `parts` pieces (streaming form; pieces given as
 * pointers and sizes). The hash of every check of the format. No reference counterpart (the reference calls the
 * vendored xxHash directly). */
uint64_t pv_xxh3_64(const void* data, uint64_t n);
uint64_t pv_xxh3_64_parts(const void* const* ptrs, const uint64_t* sizes, int32_t parts);

/* Incremental XXH3-64 (seed 0): a handle, updates with consecutive pieces, the digest of everything so far (the handle
 * stays usable), free. Equal to pv_xxh3_64 of the concatenation. No reference counterpart (the reference hashes a
 * whole host buffer at once, csrc/pv_core.cpp:167-176); the check_full pipeline needs it. */
void *pv_xxh3_stream_new(void);
void pv_xxh3_stream_update(void* h, const void* data, uint64_t n);
uint64_t pv_xxh3_stream_digest(const void* h);
void pv_xxh3_stream_free(void* h);

/* ---- device side ------------------------------------------------------------------------------------------------ */

/* The resident cohort as the kernels read it: device pointers to the pooled arrays above plus scalars. The arrays a
 * form does not use may be NULL (off / st / run0 with PV_FORM_COMPACT_BLOCKS, ref with PV_FORM_PACKED_REF, and the
 * arrays of a form not chosen). */
typedef struct pv_dev_cohort {
    const uint8_t* P;
    const uint32_t* off;
    const int64_t* st;
    const uint32_t* run0;
    const uint8_t* tab;
    const int64_t* asm_rec;     /* ASM array */
    const int64_t* low_s;
    const int64_t* low_l;
    const uint8_t* ref;
    uint64_t ref_n;
    int64_t nasm;
    uint32_t Q;
    uint32_t form;              /* PV_FORM_* bits */
    const uint32_t* pw;         /* PV_FORM_PACKED_REF */
    const int64_t* pes;
    const int64_t* pel;
    const uint8_t* peb;
    const uint32_t* peix;
    int64_t pne;
    const int64_t* grp_off;     /* PV_FORM_COMPACT_BLOCKS */
    const int64_t* grp_st;
    const uint32_t* run0g;
    const uint16_t* blen;
    const int16_t* bcode;
    const int64_t* exc_b;
    const int64_t* exc_st;
    int64_t nexc;
} pv_dev_cohort;

/* Decode windows [start[i], start[i]+W) of assembly asm[i] (offsets in the assembly's base stream) into
 * out[n, W] on the device, then lower-case runs (apply_case && !tokens), reverse complement (rc[i] != 0; rc may be
 * NULL) and tokens (A/a 0, C/c 1, G/g 2, T/t 3, else 4). asm, start, rc and out are device pointers; status is one
 * device int32 that the caller zeroed; bits PV_ST_*.
 * Launches on `stream` (a hipStream_t; NULL = the null stream) and returns without waiting.
 * work / work_bytes: optional device scratch (16-byte aligned). With at least pv_windows_work_bytes(D, n, W) bytes,
 * blocks with short payloads are decoded one lane per block by a first kernel and the windows kernel only replays
 * them; with less (or NULL) every block is decoded by the windows kernel. The bytes returned are the same.
 * Replaces _C.windows_cuda / pv_windows_cuda + run_windows (reference csrc/pv_cuda.cu:117-162), including its checks:
 * Q in {1024, 2048, 4096, 16384}, 0 <= W < 2^31, n * (ceil(W/Q)+1) < 2^31 -> PV_EARG.
 * A call that uses the work buffer refuses a stream under graph capture (PV_EARG): its list and done words carry a
 * number drawn on the host per launch, which a replayed graph would repeat. */
int32_t pv_windows_hip(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W,
                       const uint8_t* rc, int32_t tokens, int32_t apply_case, uint8_t* out, int32_t* status,
                       void* work, uint64_t work_bytes, void* stream, char* err, size_t errcap);
/* What a call of n windows of W bases on `stream` uses besides its buffers, set up ahead of the first such call: for a
 * call of more than 16,384 (window, covering block) slots (2,048 at Q = 16384), the side stream its long-block decode runs on (the heavy
 * waves at Q <= 4096; at Q = 16384 the whole-slot pass, beside the replay) and the two events that fork and join it
 * (otherwise made by the first such call on the stream). pv_windows_hip and
 * pv_sample_hip on the caller's own stream fork; pv_sample_hip on a ring stream does not (the ring overlaps calls). Idempotent; PV_OK
 * also where nothing is needed or the side stream cannot be had (such calls then run on `stream` alone). Call with
 * the stream's device current. No reference counterpart. */
int32_t pv_launch_prepare(const pv_dev_cohort* D, int64_t n, int64_t W, void* stream, char* err, size_t errcap);
/* Host check of the decode kernels' four-bytes-at-a-time output transforms (complement, complement keeping case,
 * token codes, lower-case flags) against their per-byte definitions, over every byte value: the number of mismatches
 * (0). No reference counterpart; tests call it without a GPU. */
int32_t pv_selftest_bytes(void);
/* Scratch bytes pv_windows_hip / pv_windows_ids_hip use for n windows of W bases (768 per (window, covering block)
 * slot, plus the heavy areas at Q <= 4096). No reference counterpart. */
uint64_t pv_windows_work_bytes(const pv_dev_cohort* D, int64_t n, int64_t W);

/* pv_windows_hip with no work argument and no allocation: its scratch (the light-block slots and, where they fit, the
 * heavy areas of pv_windows_work_bytes) is a file-scope device array of PV_NOALLOC_SCRATCH_BYTES that each GPU holds
 * from the first call on it until the process ends. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid hipMalloc). A stream under graph capture is
 * refused (PV_EARG) as by pv_windows_hip: a replayed graph would repeat the call's per-launch list numbers. It
 * calls no hipMalloc, hipFree or allocating library routine. Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (other streams, other threads) race; calls on one stream are ordered. Nothing in the array
 * needs to start at zero, so no call clears it. PV_EARG when n windows of W bases need more than
 * PV_NOALLOC_SCRATCH_BYTES of light-block slots (768 bytes per window x covering block: 43,690 slots, e.g. n = 14,563
 * at W = 8192, q4k); at Q = 16384 such a call runs with no scratch instead (every block by the windows kernel's wave
 * decoder). Other arguments, results and errors as pv_windows_hip. */
#define PV_NOALLOC_SCRATCH_BYTES (32u << 20)
int32_t pv_windows_hip_noalloc(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W,
                               const uint8_t* rc, int32_t tokens, int32_t apply_case, uint8_t* out, int32_t* status,
                               void* stream, char* err, size_t errcap);

/* As pv_windows_hip with tokens, but every token t (A/a 0, C/c 1, G/g 2, T/t 3, else 4) is stored as ids[t] into an
 * int64 row: out is a device i64[n, W], ids a device i64[5]. This fuses the id lookup a training loader applies to
 * the token windows (reference tools/megatron/panvram_loader.py:96-97, `lut5[raw.long()]`) into the decode's store.
 * Case runs do not apply (tokens ignore case). Errors as pv_windows_hip; PV_EARG for a NULL ids. */
int32_t pv_windows_ids_hip(const pv_dev_cohort* D, const int64_t* asm_idx, const int64_t* start, int64_t n, int64_t W, const uint8_t* rc,
                           const int64_t* ids, int64_t* out, int32_t* status, void* work, uint64_t work_bytes, void* stream, char* err,
                           size_t errcap);

/* One window of W bases at base `start` of assembly `assembly`'s base stream, the coordinates passed by value: what
 * Cohort.fetch does with pv_windows_hip on one-element tensors (reference panvram/cohort.py:196-207), without the two
 * host-to-device copies of those tensors and the fill of the status word. `rec` is device memory of 32 bytes, 16-byte
 * aligned: the call's first kernel on `stream` writes the assembly (i64, byte 0), the start (i64, byte 8) and the
 * strand (u8, byte 16; rc != 0 reverse-complements) there and zeroes the int32 status word at byte 24, which the
 * decode then sets as pv_windows_hip's status (with a work buffer below 16 K block size the decode kernel itself,
 * which takes the coordinates as arguments; otherwise a small kernel of its own first). out: u8[W]; apply_case is on. work, errors and the rest as pv_windows_hip with n = 1.
 * Consecutive calls may reuse `rec` on one stream (the launches are ordered). No reference counterpart as a C
 * function. */
int32_t pv_fetch_hip(const pv_dev_cohort* D, int64_t assembly, int64_t start, int64_t W, int32_t rc, int32_t tokens,
                     uint8_t* out, void* rec, void* work, uint64_t work_bytes, void* stream, char* err, size_t errcap);

/* Window coordinates of Cohort.sample's random draws, one launch on `stream` (the torch searchsorted / gather / add
 * steps of the reference's Cohort.sample, panvram/cohort.py:177-189, in one kernel; no reference counterpart as a
 * function). The windows are then decoded with pv_windows_hip(wasm, wstart, wrc).
 *  cum        i64[ncontigs] per-W running count of valid window starts (cumsum of max(0, contig length - W + 1))
 *  ctg_*      i64[ncontigs] contig tables (PV_ARR_CTG_*, on the device)
 *  draws      i64[n]        torch.randint(0, cum[ncontigs-1], (n,)) draws
 *  rnd, p     f32[n], p     rcmode 2: window i reverse-complemented iff rnd[i] < (float)p; rcmode 1: all; 0: none
 *  wasm, wstart i64[n]      out: assembly and start in its base stream (-1: a draw past the table)
 *  wrc        u8[n]         out (rcmode 1, 2): strand
 *  coords     i64[n, 4] or NULL: out (assembly, contig index, start in the contig, strand)
 *  status     int32, zeroed by the kernel (no separate memset)
 * Errors: PV_EARG, PV_EHIP. */
int32_t pv_sample_coords_hip(const int64_t* cum, int64_t ncontigs, const int64_t* ctg_asm, const int64_t* ctg_local,
                             const int64_t* ctg_boff, const int64_t* draws, const float* rnd, double p, int32_t rcmode, int64_t n,
                             int64_t* wasm, int64_t* wstart, uint8_t* wrc, int64_t* coords, int32_t* status, void* stream,
                             char* err, size_t errcap);

/* How pv_sample_hip makes the caller's stream wait for the lane stream. */
#define PV_WAIT_EVENT 0     /* an event from a ring the library keeps per device (hipStreamWaitEvent) */
#define PV_WAIT_COUNTER 1   /* a counter per lane stream in signal memory (hipStreamWriteValue64 / hipStreamWaitValue64):
                               less host time per call; the runtime waits with a polling kernel on the caller's queue,
                               so not for use where dispatches are serialised (rocprofv3 --pmc), where it stalls */

/* Cohort.sample after its draws, in one call: pv_sample_coords_hip and pv_windows_hip on `stream`, then `caller` (a
 * hipStream_t; NULL is HIP's null stream) made to wait for both, unless it is `stream` itself, the way `wait` says
 * (PV_WAIT_COUNTER falls back to events where the device lacks stream wait-value support, or under a tool that
 * serialises dispatches, pv_dispatch_serialised). Calls on one device are serialised by a mutex from their first launch
 * to the wait. With a `stream` other than `caller`, the caller's stream marks its progress after its wait, and a call
 * first waits on the host until the caller's stream has passed all but 31 of its earlier calls (PV_EHIP after 60 s
 * without progress): at most 32 calls (and what their callers free after them) are in flight per caller stream. ev_start / ev_mid / ev_end: hipEvent_t on `stream`, or
 * NULL: ev_start is recorded just before the decode launches; given both, ev_mid and ev_end are set to the windows
 * (replay and write-out) kernel's own start and end (hipExtLaunchKernel), else each is recorded just before / after it.
 * work: 16-byte aligned device scratch of work_bytes >=
 * pv_sample_work_bytes(D, n, W): the windows' assembly, start and strand (17 n bytes, rounded up to 256), then the
 * scratch of pv_windows_hip. ids: NULL (out: u8[n, W] as for
 * pv_windows_hip) or a device i64[5] (out: i64[n, W] token ids as for pv_windows_ids_hip). Other arguments and errors as
 * for pv_sample_coords_hip and pv_windows_hip. No reference counterpart as a function (it replaces the torch ops of the
 * reference's Cohort.sample, panvram/cohort.py:177-190, and its windows call). */
int32_t pv_sample_hip(const pv_dev_cohort* D, const int64_t* cum, int64_t ncontigs, const int64_t* ctg_asm, const int64_t* ctg_local,
                      const int64_t* ctg_boff, const int64_t* draws, const float* rnd, double p, int32_t rcmode, int64_t n, int64_t W,
                      int32_t tokens, int32_t apply_case, const int64_t* ids, void* work, uint64_t work_bytes, int64_t* coords,
                      void* out, int32_t* status, void* stream, void* caller, int32_t wait, void* ev_start, void* ev_mid,
                      void* ev_end, char* err, size_t errcap);
/* pv_sample_hip's arguments as one record, so that a binding which calls it repeatedly with mostly the same arguments
 * (a Python loader: only `out` and `coords` change between calls on one stream) passes one pointer instead of 28
 * converted arguments. */
typedef struct pv_sample_call {
    const pv_dev_cohort* D;
    const int64_t* cum; int64_t ncontigs; const int64_t* ctg_asm; const int64_t* ctg_local; const int64_t* ctg_boff;
    const int64_t* draws; const float* rnd; double p; int32_t rcmode; int32_t tokens; int64_t n; int64_t W;
    int32_t apply_case; int32_t wait; const int64_t* ids; void* work; uint64_t work_bytes; int64_t* coords; void* out;
    int32_t* status; void* stream; void* caller; void* ev_start; void* ev_mid; void* ev_end; char* err; uint64_t errcap;
} pv_sample_call;
/* pv_sample_hip(c->D, c->cum, ..., c->err, c->errcap). No reference counterpart (a calling convention of pv_sample_hip). */
int32_t pv_sample_hip_call(const pv_sample_call* c);
/* Bytes of pv_sample_hip's `work` for n windows of W bases. No reference counterpart. */
uint64_t pv_sample_work_bytes(const pv_dev_cohort* D, int64_t n, int64_t W);
/* What pv_sample_hip's waits need for lane stream `stream` and caller stream `caller`, set up before the first call on
 * them, so that no later call allocates or synchronises: their events, and for PV_WAIT_COUNTER their counters in signal
 * memory (zeroed, the stream synchronised once). Call with their device current. No reference counterpart (the
 * reference's sample runs on the caller's stream). */
int32_t pv_sample_prepare(void* stream, void* caller, int32_t wait, char* err, size_t errcap);
/* sample's rows from a pool of the library's own, handed to torch as DLPack tensors (DLManagedTensor, device type
 * ROCm): a row torch frees is handed out again once the caller's stream has passed the next call's wait, so the caller's
 * queue needs no allocator event per call. pv_rows_reserve: the current device's pool of `bytes`-byte rows, grown to at
 * least `count` rows (hipMalloc; the process's pools hold 4 GiB of rows at most, and idle rows of the device's other
 * pools are freed first to make room; fewer where that or the device's memory runs out) - set-up, before the calls
 * (hipFree synchronises the device). No reference
 * counterpart (the reference's rows come from torch's allocator, csrc/pv_cuda.cu:123). */
int32_t pv_rows_reserve(uint64_t bytes, int32_t count, void** pool, char* err, size_t errcap);
/* A row for an n x W tensor of `bits`-bit elements (8: uint8, 64: int64) for caller stream `caller` (one that
 * pv_sample_prepare set up with PV_WAIT_COUNTER), as a DLManagedTensor* whose deleter returns it to the pool; NULL when
 * no row is free yet (the caller then allocates its own). No reference counterpart. */
void* pv_rows_take(void* pool, void* caller, int64_t n, int64_t W, int32_t bits);
/* The pool's rows and those not handed out. No reference counterpart. */
int32_t pv_rows_count(const void* pool, int32_t* total, int32_t* free_rows);
/* 1 when the process runs under a tool that serialises kernel dispatches (rocprofv3 counter collection or thread
 * trace, read from the environment it sets), where PV_WAIT_COUNTER behaves as PV_WAIT_EVENT. No reference counterpart. */
int32_t pv_dispatch_serialised(void);
/* Whether work on streams a and b (hipStream_t) runs at the same time: HIP maps a process's streams onto its
 * GPU_MAX_HW_QUEUES hardware queues (4 by default), several streams to a queue when there are more streams, and kernels
 * on one queue run one after another. Both streams are synchronised, then a one-wave kernel that waits 100 us of the
 * GPU's real-time clock is launched on each, released together by an event; *concurrent = 1 when the two end within
 * 1.5 times one kernel's time of the release. Set-up only (it synchronises). No reference counterpart (the host layer
 * picks sample's ring streams with it at up to 8 hardware queues, so that they do not share a queue with each other or
 * with the caller). */
int32_t pv_streams_concurrent(void* a, void* b, int32_t* concurrent, char* err, size_t errcap);

/* FASTA bytes [f0, f0 + nf) of one assembly into out (device), laid out from its decoded bases [b0, b0 + nb) (device,
 * case applied): per record '>' header '\n', then lines of line-width bases each ended by '\n' - the layout of the
 * reference's Core::fasta (csrc/pv_core.cpp:138-159). rec: device i64[nrec * 6] = {FASTA offset, header offset in
 * hdrs, header length, length, base-stream offset, line width} per record, in file order; hdrs: device header bytes.
 * One launch on `stream`. No reference counterpart as a function (the reference builds the file on the host). */
int32_t pv_fasta_layout_hip(const uint8_t* bases, uint64_t b0, uint64_t nb, const int64_t* rec, int32_t nrec, const uint8_t* hdrs,
                            uint64_t f0, uint64_t nf, uint8_t* out, void* stream, char* err, size_t errcap);

#ifdef __cplusplus
}
#endif
#endif
