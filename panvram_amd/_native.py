"""ctypes binding of libpanvram_amd.so (declarations in include/panvram_amd.h).

The library links the HIP runtime by its SONAME; torch is imported first so that the runtime torch already loaded is
the one the library binds to (same streams, same device pointers). A missing library is an ImportError: the package
has no CPU fallback.
"""
import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library shares)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpanvram_amd.so")

PV_OK, PV_EFORMAT, PV_EARG, PV_EHIP, PV_ENOMEM = 0, 1, 2, 3, 4
(ARR_P, ARR_OFF, ARR_ST, ARR_RUN0, ARR_TAB, ARR_ASM, ARR_LOW_S, ARR_LOW_L, ARR_REF,
 ARR_CTG_ASM, ARR_CTG_LOCAL, ARR_CTG_BOFF, ARR_CTG_LEN,
 ARR_PW, ARR_PES, ARR_PEL, ARR_PEB, ARR_PEIX,
 ARR_GRP_OFF, ARR_GRP_ST, ARR_RUN0G, ARR_BLEN, ARR_BCODE, ARR_EXC_B, ARR_EXC_ST, ARR_COUNT) = range(26)
FORM_PACKED_REF, FORM_COMPACT_BLOCKS = 1, 2
WAIT_EVENT, WAIT_COUNTER = 0, 1

vp, i32, i64, u32, u64, cp, sz = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64,
                                  ctypes.c_char_p, ctypes.c_size_t)


class FormatError(ValueError):
    """A refused archive or reference, or a corrupt block (the reference's panvram.FormatError, a ValueError)."""


class AsmInfo(ctypes.Structure):
    _fields_ = [("Q", u32), ("flags", u32), ("bases", u64), ("blocks", u64), ("file_bytes", u64), ("payload_bytes", u64),
                ("contigs", u64), ("lower_case_runs", u64), ("fasta_xxh3", u64), ("bases_xxh3", u64), ("block_hashes", i32),
                ("path", ctypes.c_char * 1024), ("reference_name", ctypes.c_char * 512)]


class DevCohort(ctypes.Structure):
    _fields_ = [("P", vp), ("off", vp), ("st", vp), ("run0", vp), ("tab", vp), ("asm_rec", vp), ("low_s", vp), ("low_l", vp),
                ("ref", vp), ("ref_n", u64), ("nasm", i64), ("Q", u32), ("form", u32),
                ("pw", vp), ("pes", vp), ("pel", vp), ("peb", vp), ("peix", vp), ("pne", i64),
                ("grp_off", vp), ("grp_st", vp), ("run0g", vp), ("blen", vp), ("bcode", vp), ("exc_b", vp), ("exc_st", vp),
                ("nexc", i64)]


class SampleCall(ctypes.Structure):
    """pv_sample_call: pv_sample_hip's arguments as one record (pv_sample_hip_call)."""
    _fields_ = [("D", vp), ("cum", vp), ("ncontigs", i64), ("ctg_asm", vp), ("ctg_local", vp), ("ctg_boff", vp),
                ("draws", vp), ("rnd", vp), ("p", ctypes.c_double), ("rcmode", i32), ("tokens", i32), ("n", i64), ("W", i64),
                ("apply_case", i32), ("wait", i32), ("ids", vp), ("work", vp), ("work_bytes", u64), ("coords", vp), ("out", vp),
                ("status", vp), ("stream", vp), ("caller", vp), ("ev_start", vp), ("ev_mid", vp), ("ev_end", vp), ("err", vp),
                ("errcap", u64)]


# every exported symbol of include/panvram_amd.h with its signature: name -> (restype, argtypes)
SIGNATURES = {
    "pv_abi_version": (i32, []),
    "pv_cohort_open": (i32, [cp, vp, i32, i32, i32, ctypes.POINTER(vp), cp, sz]),
    "pv_cohort_form": (i32, [vp]),
    "pv_cohort_ref_exceptions": (i64, [vp]),
    "pv_cohort_block_exceptions": (i64, [vp]),
    "pv_cohort_close": (None, [vp]),
    "pv_cohort_block_size": (i32, [vp]),
    "pv_cohort_assemblies": (i64, [vp]),
    "pv_cohort_ref_bases": (u64, [vp]),
    "pv_cohort_ref_sha256": (None, [vp, cp]),
    "pv_cohort_array": (i32, [vp, i32, ctypes.POINTER(vp), ctypes.POINTER(u64)]),
    "pv_cohort_release_array": (i32, [vp, i32]),
    "pv_asm_info_get": (i32, [vp, i64, ctypes.POINTER(AsmInfo)]),
    "pv_asm_contig": (i32, [vp, i64, i64, ctypes.POINTER(cp), ctypes.POINTER(cp), ctypes.POINTER(u64), ctypes.POINTER(u64), ctypes.POINTER(u32)]),
    "pv_fasta_xxh3": (i32, [vp, i64, vp, u64, ctypes.POINTER(u64), cp, sz]),
    "pv_fasta_size": (u64, [vp, i64]),
    "pv_fasta_build": (i32, [vp, i64, vp, u64, vp, u64, cp, sz]),
    "pv_verify_blocks": (i32, [vp, i64, vp, u64, ctypes.POINTER(i64)]),
    "pv_apply_case": (i32, [vp, i64, u64, vp, u64]),
    "pv_sha256_file_bases": (i32, [cp, cp, cp, sz]),
    "pv_xxh3_64": (u64, [vp, u64]),
    "pv_xxh3_64_parts": (u64, [vp, vp, i32]),
    "pv_windows_hip": (i32, [ctypes.POINTER(DevCohort), vp, vp, i64, i64, vp, i32, i32, vp, vp, vp, u64, vp, cp, sz]),
    "pv_windows_work_bytes": (u64, [ctypes.POINTER(DevCohort), i64, i64]),
    "pv_sample_work_bytes": (u64, [ctypes.POINTER(DevCohort), i64, i64]),
    "pv_sample_coords_hip": (i32, [vp, i64, vp, vp, vp, vp, vp, ctypes.c_double, i32, i64, vp, vp, vp, vp, vp, vp, cp, sz]),
    "pv_xxh3_stream_new": (vp, []),
    "pv_xxh3_stream_update": (None, [vp, vp, u64]),
    "pv_xxh3_stream_digest": (u64, [vp]),
    "pv_xxh3_stream_free": (None, [vp]),
    "pv_fasta_layout_hip": (i32, [vp, u64, u64, vp, i32, vp, u64, u64, vp, vp, cp, sz]),
    "pv_sample_hip": (i32, [ctypes.POINTER(DevCohort), vp, i64, vp, vp, vp, vp, vp, ctypes.c_double, i32, i64, i64, i32, i32,
                            vp, vp, u64, vp, vp, vp, vp, vp, i32, vp, vp, vp, cp, sz]),
    "pv_sample_hip_call": (i32, [ctypes.POINTER(SampleCall)]),
    "pv_sample_prepare": (i32, [vp, vp, i32, cp, sz]),
    "pv_launch_prepare": (i32, [vp, i64, i64, vp, cp, sz]),
    "pv_rows_reserve": (i32, [u64, i32, ctypes.POINTER(vp), cp, sz]),
    "pv_rows_take": (vp, [vp, vp, i64, i64, i32]),
    "pv_rows_count": (i32, [vp, ctypes.POINTER(i32), ctypes.POINTER(i32)]),
    "pv_dispatch_serialised": (i32, []),
    "pv_streams_concurrent": (i32, [vp, vp, ctypes.POINTER(i32), cp, sz]),
    "pv_windows_ids_hip": (i32, [ctypes.POINTER(DevCohort), vp, vp, i64, i64, vp, vp, vp, vp, vp, u64, vp, cp, sz]),
    "pv_windows_hip_noalloc": (i32, [ctypes.POINTER(DevCohort), vp, vp, i64, i64, vp, i32, i32, vp, vp, vp, cp, sz]),
    "pv_selftest_bytes": (i32, []),
    "pv_fetch_hip": (i32, [ctypes.POINTER(DevCohort), i64, i64, i64, i32, i32, vp, vp, vp, u64, vp, cp, sz]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build() (hipcc for gfx950); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def errbuf():
    return ctypes.create_string_buffer(4096)


def raise_for(code, err, default=RuntimeError):
    msg = err.value.decode(errors="replace") if err is not None else ""
    if code == PV_EFORMAT:
        raise FormatError(msg)
    if code == PV_ENOMEM:
        raise MemoryError(msg)
    raise default(msg or f"panvram_amd error {code}")
