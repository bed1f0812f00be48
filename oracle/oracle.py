"""ctypes binding of the fp64 CPU oracle (oracle/pdattn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()`` as the checker and
by the CPU-baseline leg of ``bench.py``. The product library never loads it.

Each wrapper names the reference function it restates (qilem/cuda-kernel-lab,
01_decode_attention.cu); the C file carries the same citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HEAD_DIM = 128
PAGE = 16

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

FAULTS = {
    "none": 0,
    "page_off_by_one": 1,
    "kvh_modulo": 2,
    "no_scale": 3,
    "full_last_page": 4,
    "lse_no_max": 5,
    "slot_transpose": 6,
    "merge_no_weight": 7,
    "half_trunc": 8,
    "prefix_no_private": 9,
}


def build(force: bool = False) -> str:
    """Compile the oracle with gcc (oracle/Makefile) and return the library path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE] + (["-B"] if force else []), check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i, d = ctypes.c_int, ctypes.c_double
        L.oracle_half_to_double.argtypes = [ctypes.c_uint16]
        L.oracle_half_to_double.restype = d
        L.oracle_double_to_half.argtypes = [d]
        L.oracle_double_to_half.restype = ctypes.c_uint16
        L.oracle_decode_mt.argtypes = [P] * 6 + [i, i, i, i, d, P, P, i]
        L.oracle_decode_mt.restype = None
        L.oracle_partials.argtypes = [P] * 6 + [i] * 8 + [d, P, P]
        L.oracle_partials.restype = None
        L.oracle_merge.argtypes = [P, P, i, i, P, P]
        L.oracle_merge.restype = None
        L.oracle_shared_prefix_pages.argtypes = [P, P, i]
        L.oracle_shared_prefix_pages.restype = i
        L.oracle_plan_chunks_ref.argtypes = [i, i, i, i, i, ctypes.POINTER(i), ctypes.POINTER(i)]
        L.oracle_plan_chunks_ref.restype = None
        L.oracle_set_fault.argtypes = [i]
        L.oracle_set_fault.restype = None
        _lib = L
    return _lib


class fault:
    """Context manager that plants one named mistake in the oracle (test use only)."""

    def __init__(self, name: str):
        self.code = FAULTS[name]

    def __enter__(self):
        lib().oracle_set_fault(self.code)
        return self

    def __exit__(self, *exc):
        lib().oracle_set_fault(0)
        return False


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a, dtype=np.uint16)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.int32)


def half_to_double(bits: int) -> float:
    return lib().oracle_half_to_double(int(bits))


def double_to_half(x: float) -> int:
    return lib().oracle_double_to_half(float(x))


def decode(q, k, v, indptr, indices, last, Hq: int, Hkv: int, kv_start: int = 0,
           sm_scale: float | None = None, threads: int = 1):
    """fp64 decode attention over the paged cache (01_decode_attention.cu:370-400).

    Returns (out [B, Hq, 128] float64, lse [B, Hq] float64)."""
    q, k, v = _u16(q), _u16(k), _u16(v)
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    B = len(indptr) - 1
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(HEAD_DIM)
    if indices.size == 0:
        indices = np.zeros(1, np.int32)
    out = np.zeros((B, Hq, HEAD_DIM), np.float64)
    lse = np.zeros((B, Hq), np.float64)
    lib().oracle_decode_mt(_ptr(q), _ptr(k), _ptr(v), _ptr(indptr), _ptr(indices), _ptr(last),
                           B, Hq, Hkv, kv_start, float(sm_scale), _ptr(out), _ptr(lse), int(threads))
    return out, lse


def partials(q, k, v, indptr, indices, last, Hq: int, Hkv: int, num_chunks: int,
             chunk_tokens: int, kv_start: int = 0, sm_scale: float | None = None):
    """Per-chunk normalized partial states with uniform chunks (01_decode_attention.cu:88-97,
    228-235). Returns (part_o [B*Hq, num_chunks, 128], part_lse [B*Hq, num_chunks])."""
    q, k, v = _u16(q), _u16(k), _u16(v)
    indptr, indices, last = _i32(indptr), _i32(indices), _i32(last)
    B = len(indptr) - 1
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(HEAD_DIM)
    if indices.size == 0:
        indices = np.zeros(1, np.int32)
    po = np.zeros((B * Hq, num_chunks, HEAD_DIM), np.float64)
    pl = np.zeros((B * Hq, num_chunks), np.float64)
    lib().oracle_partials(_ptr(q), _ptr(k), _ptr(v), _ptr(indptr), _ptr(indices), _ptr(last),
                          B, Hq, Hkv, num_chunks, chunk_tokens, kv_start, 0, num_chunks,
                          float(sm_scale), _ptr(po), _ptr(pl))
    return po, pl


def merge(part_o, part_lse):
    """Log-sum-exp merge over the chunk axis (01_decode_attention.cu:238-255).

    part_o [rows, C, 128], part_lse [rows, C] -> (out [rows, 128], lse [rows])."""
    po = np.ascontiguousarray(part_o, dtype=np.float64)
    pl = np.ascontiguousarray(part_lse, dtype=np.float64)
    rows, C = pl.shape
    out = np.zeros((rows, HEAD_DIM), np.float64)
    lse = np.zeros(rows, np.float64)
    lib().oracle_merge(_ptr(po), _ptr(pl), rows, C, _ptr(out), _ptr(lse))
    return out, lse


def shared_prefix_pages(indptr, indices) -> int:
    """Longest shared run of leading physical pages, one private page kept
    (01_decode_attention.cu:634-646)."""
    indptr, indices = _i32(indptr), _i32(indices)
    if indices.size == 0:
        indices = np.zeros(1, np.int32)
    return int(lib().oracle_shared_prefix_pages(_ptr(indptr), _ptr(indices), len(indptr) - 1))


def plan_chunks_ref(resident_blocks: int, B: int, Hkv: int, max_len: int, force_chunks: int = 0):
    """The reference's uniform chunk rule (01_decode_attention.cu:289-312)."""
    nc, ct = ctypes.c_int(), ctypes.c_int()
    lib().oracle_plan_chunks_ref(resident_blocks, B, Hkv, max_len, force_chunks,
                                 ctypes.byref(nc), ctypes.byref(ct))
    return nc.value, ct.value


APPEND_FAULTS = ("none", "slot_kvh_transpose", "page_off_by_one", "position_minus_one")


def append_kv(k_cache, v_cache, k_new, v_new, batch_idx, positions, indptr, indices,
              fault: str = "none"):
    """Paged KV append, restated on the host: token t, at position p of sequence b, is written to
    page indices[indptr[b] + p // 16], slot p % 16, for every kv head -- the page addressing of
    01_decode_attention.cu:112 used for writes (FlashInfer's append convention: the page table
    already covers the appended tokens). Tokens whose sequence or position is out of range are
    skipped and counted. Caches are [num_pages, 16, Hkv, 128] (any 2-byte dtype), new rows
    [n, Hkv, 128]. `fault` plants a mistake for the tests that pin this function.

    Returns (k_cache', v_cache', n_invalid)."""
    kc, vc = np.array(k_cache, copy=True), np.array(v_cache, copy=True)
    indptr, indices = np.asarray(indptr), np.asarray(indices)
    B = len(indptr) - 1
    bad = 0
    for t in range(len(batch_idx)):
        b, p = int(batch_idx[t]), int(positions[t])
        if fault == "position_minus_one":
            p -= 1
        if b < 0 or b >= B or p < 0 or p >= (indptr[b + 1] - indptr[b]) * PAGE:
            bad += 1
            continue
        j = indptr[b] + p // PAGE + (1 if fault == "page_off_by_one" else 0)
        j = min(j, len(indices) - 1)
        page, slot = int(indices[j]), p % PAGE
        if fault == "slot_kvh_transpose":
            # rows laid out [kvh][slot] instead of [slot][kvh]
            flat_k, flat_v = kc[page].reshape(-1, HEAD_DIM), vc[page].reshape(-1, HEAD_DIM)
            Hkv = kc.shape[2]
            for h in range(Hkv):
                flat_k[(h * PAGE + slot) % (PAGE * Hkv)] = k_new[t, h]
                flat_v[(h * PAGE + slot) % (PAGE * Hkv)] = v_new[t, h]
            continue
        kc[page, slot] = k_new[t]
        vc[page, slot] = v_new[t]
    return kc, vc, bad

