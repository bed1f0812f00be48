"""ctypes binding of libpdattn (include/pdattn.h) for Python callers, tests and the benchmark.

This is the Python face of the C ABI: every function maps 1:1 onto an ``extern "C"`` entry point
and raises ``PdattnError`` on a non-zero status. Device memory is passed as integers (device
addresses) or as any object with ``data_ptr()`` (e.g. a torch tensor); streams as integers
(a hipStream_t) or objects with ``cuda_stream``. The compute itself is always the HIP library:
there is no fallback, and loading fails loudly if the library has not been built.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

HEAD_DIM = 128
PAGE = 16

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG_DIR)
LIB_PATH = os.path.join(_ROOT, "lib", "libpdattn.so")

_lib = None

STATUS = {
    0: "PDATTN_OK",
    1: "PDATTN_ERR_INVALID_ARGUMENT",
    2: "PDATTN_ERR_UNSUPPORTED",
    3: "PDATTN_ERR_PAGE_TABLE",
    4: "PDATTN_ERR_WORKSPACE",
    5: "PDATTN_ERR_HIP",
    6: "PDATTN_ERR_NOT_READY",
}

# Every symbol include/pdattn.h declares.
EXPORTS = [
    "pdattn_strerror", "pdattn_last_error",
    "pdattn_workspace_reserve", "pdattn_workspace_release",
    "pdattn_check_page_table",
    "pdattn_plan_chunks", "pdattn_decode_partial", "pdattn_merge_states",
    "pdattn_decode_workspace_size", "pdattn_workspace_partials", "pdattn_decode_attention",
    "pdattn_decode_attention_noalloc", "pdattn_decode_attention_balanced",
    "pdattn_decode_balanced_workspace_size",
    "pdattn_plan_create", "pdattn_plan_get_info", "pdattn_plan_workspace_size",
    "pdattn_plan_get_schedule", "pdattn_plan_upload", "pdattn_plan_run", "pdattn_plan_run_part",
    "pdattn_plan_destroy",
    "pdattn_shared_prefix_pages", "pdattn_cascade_prefix",
    "pdattn_cascade_plan_create", "pdattn_cascade_tree_plan_create", "pdattn_cascade_plan_get_info",
    "pdattn_cascade_decode", "pdattn_cascade_set_mode",
    "pdattn_cascade_plan_destroy",
    "pdattn_append_kv",
    "pdattn_stream_read", "pdattn_flush_cache", "pdattn_get_device_info",
]


class PdattnError(RuntimeError):
    def __init__(self, status: int, where: str, detail: str):
        self.status = status
        super().__init__(f"{where}: {STATUS.get(status, status)}: {detail}")


class DecodeParams(ctypes.Structure):
    """pdattn_decode_params (mirrors DecodeParams, 01_decode_attention.cu:51-65)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("kv_indptr", ctypes.c_void_p), ("kv_indices", ctypes.c_void_p),
        ("kv_last_page_len", ctypes.c_void_p),
        ("part_o", ctypes.c_void_p), ("part_lse", ctypes.c_void_p),
        ("B", ctypes.c_int32), ("Hq", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("num_chunks", ctypes.c_int32), ("chunk_tokens", ctypes.c_int32),
        ("kv_start", ctypes.c_int32), ("chunk_base", ctypes.c_int32),
        ("part_stride", ctypes.c_int32), ("sm_scale", ctypes.c_float),
    ]


class Workspace(ctypes.Structure):
    """pdattn_workspace (replaces Workspace, 01_decode_attention.cu:314)."""
    _fields_ = [("base", ctypes.c_void_p), ("bytes", ctypes.c_size_t), ("owned", ctypes.c_int)]


class PrefixParams(ctypes.Structure):
    """pdattn_prefix_params (mirrors PrefixParams, 01_decode_attention.cu:473-482)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("prefix_pages", ctypes.c_void_p), ("part_o", ctypes.c_void_p),
        ("part_lse", ctypes.c_void_p),
        ("B", ctypes.c_int32), ("Hq", ctypes.c_int32), ("Hkv", ctypes.c_int32),
        ("prefix_len", ctypes.c_int32), ("chunk_tokens", ctypes.c_int32),
        ("part_stride", ctypes.c_int32), ("sm_scale", ctypes.c_float),
    ]


class PlanInfo(ctypes.Structure):
    _fields_ = [("workgroups", ctypes.c_int), ("pairs", ctypes.c_int),
                ("split_pairs", ctypes.c_int), ("max_contributors", ctypes.c_int),
                ("units", ctypes.c_int64), ("workspace_bytes", ctypes.c_size_t),
                ("chunk_pages", ctypes.c_int), ("segments", ctypes.c_int),
                ("merge_entries", ctypes.c_int), ("schedule_ints", ctypes.c_int),
                ("paired", ctypes.c_int)]


class CascadeInfo(ctypes.Structure):
    _fields_ = [("use", ctypes.c_int), ("prefix_tokens", ctypes.c_int),
                ("prefix_chunks", ctypes.c_int), ("prefix_workgroups", ctypes.c_int),
                ("suffix_workgroups", ctypes.c_int), ("workspace_bytes", ctypes.c_size_t),
                ("nodes", ctypes.c_int), ("levels", ctypes.c_int), ("mode", ctypes.c_int)]


# pdattn_cascade_set_mode
CASCADE_FUSED, CASCADE_SERIAL, CASCADE_TWO_STREAMS = 0, 1, 2
RUN_DECODE, RUN_MERGE, RUN_ALL = 1, 2, 3   # pdattn_plan_run_part


class DeviceInfo(ctypes.Structure):
    _fields_ = [("compute_units", ctypes.c_int), ("decode_wg_per_cu", ctypes.c_int),
                ("prefix_wg_per_cu", ctypes.c_int), ("arch", ctypes.c_char * 64)]


def build(force: bool = True) -> str:
    """Compile libpdattn.so for gfx950 with hipcc (cuda-kernel-lab_amd/Makefile)."""
    args = ["make", "-C", _ROOT, "-j8"]
    if force:
        args.append("-B")
    subprocess.run(args, check=True)
    return LIB_PATH


def lib():
    """Load libpdattn.so (raises if it has not been built: there is no fallback path)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() or "
                           f"`make -C {_ROOT}`")
    L = ctypes.CDLL(LIB_PATH)
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    sig = {
        "pdattn_strerror": ([I], ctypes.c_char_p),
        "pdattn_last_error": ([], ctypes.c_char_p),
        "pdattn_workspace_reserve": ([ctypes.POINTER(Workspace), S], I),
        "pdattn_workspace_release": ([ctypes.POINTER(Workspace)], None),
        "pdattn_check_page_table": ([P, P, P, I, ctypes.c_int64], I),
        "pdattn_plan_chunks": ([I, I, I, I, I, I, ctypes.POINTER(I), ctypes.POINTER(I)], I),
        "pdattn_decode_partial": ([ctypes.POINTER(DecodeParams), I, I, P], I),
        "pdattn_merge_states": ([P, P, P, P, I, I, P], I),
        "pdattn_decode_workspace_size": ([I, I, I], S),
        "pdattn_workspace_partials": ([ctypes.POINTER(Workspace), I, I, I,
                                       ctypes.POINTER(P), ctypes.POINTER(P)], I),
        "pdattn_decode_attention": ([ctypes.POINTER(DecodeParams), I, I, P, P,
                                     ctypes.POINTER(Workspace), P], I),
        "pdattn_decode_attention_noalloc": ([ctypes.POINTER(DecodeParams), I, I, P, P, P], I),
        "pdattn_decode_attention_balanced": ([ctypes.POINTER(DecodeParams), I, I, P, P,
                                              ctypes.POINTER(Workspace), P], I),
        "pdattn_decode_balanced_workspace_size": ([ctypes.POINTER(DecodeParams), I], S),
        "pdattn_plan_create": ([P, P, I, I, I, I, I, ctypes.POINTER(P)], I),
        "pdattn_plan_get_info": ([P, ctypes.POINTER(PlanInfo)], I),
        "pdattn_plan_get_schedule": ([P, P, S], I),
        "pdattn_plan_workspace_size": ([P], S),
        "pdattn_plan_upload": ([P, P, S, P], I),
        "pdattn_plan_run": ([P, P, P, P, P, P, P, ctypes.c_float, P, P, P, S, P], I),
        "pdattn_plan_run_part": ([P, P, P, P, P, P, P, ctypes.c_float, P, P, P, S, P, I], I),
        "pdattn_plan_destroy": ([P], None),
        "pdattn_shared_prefix_pages": ([P, P, I], I),
        "pdattn_cascade_prefix": ([ctypes.POINTER(PrefixParams), P], I),
        "pdattn_cascade_plan_create": ([ctypes.POINTER(DecodeParams), P, P, P, P, I,
                                        ctypes.POINTER(P)], I),
        "pdattn_cascade_tree_plan_create": ([ctypes.POINTER(DecodeParams), P, P, P, P, I,
                                             ctypes.POINTER(P)], I),
        "pdattn_cascade_plan_get_info": ([P, ctypes.POINTER(CascadeInfo)], I),
        "pdattn_cascade_decode": ([P, P, P, ctypes.POINTER(Workspace), P], I),
        "pdattn_cascade_set_mode": ([P, I], I),
        "pdattn_cascade_plan_destroy": ([P], None),
        "pdattn_append_kv": ([P, P, P, P, P, P, P, P, I, I, I, P, P], I),
        "pdattn_stream_read": ([P, S, P, P], I),
        "pdattn_flush_cache": ([P, S, P], I),
        "pdattn_get_device_info": ([ctypes.POINTER(DeviceInfo)], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _check(status: int, where: str):
    if status != 0:
        detail = lib().pdattn_last_error().decode(errors="replace")
        raise PdattnError(status, where, detail)


def ptr(x) -> int | None:
    """Device address of x: an int, None, or an object with data_ptr()."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


def stream_ptr(s) -> int | None:
    if s is None or isinstance(s, int):
        return s
    return int(s.cuda_stream)


def host_i32(a):
    """Contiguous int32 numpy copy of a host array and its ctypes pointer."""
    import numpy as np
    arr = np.ascontiguousarray(np.asarray(a), dtype=np.int32)
    if arr.size == 0:
        arr = np.zeros(1, np.int32)
    return arr, arr.ctypes.data_as(ctypes.c_void_p)


def check_page_table(kv_indptr, kv_indices, kv_last_page_len, num_pages: int):
    """pdattn_check_page_table on host copies of a page table: raises PdattnError
    (PDATTN_ERR_PAGE_TABLE) for a decreasing indptr, a page id outside [0, num_pages) or a last
    page length outside [1, 16]."""
    ip, ipp = host_i32(kv_indptr)
    ix, ixp = host_i32(kv_indices)
    la, lap = host_i32(kv_last_page_len)
    B = len(ip) - 1 if len(kv_indptr) > 0 else 0
    _check(lib().pdattn_check_page_table(ipp, ixp, lap, B, int(num_pages)), "pdattn_check_page_table")


# ---- reference-shaped split-KV path ------------------------------------------------------------

def plan_chunks(G: int, B: int, Hkv: int, max_len: int, force_chunks: int = 0, variant: int = 0):
    nc, ct = ctypes.c_int(), ctypes.c_int()
    _check(lib().pdattn_plan_chunks(G, variant, B, Hkv, max_len, force_chunks,
                                    ctypes.byref(nc), ctypes.byref(ct)), "pdattn_plan_chunks")
    return nc.value, ct.value


def make_params(q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, B, Hq, Hkv,
                num_chunks=1, chunk_tokens=16, kv_start=0, chunk_base=0, part_stride=None,
                sm_scale=None, part_o=None, part_lse=None) -> DecodeParams:
    p = DecodeParams()
    p.q, p.k_cache, p.v_cache = ptr(q), ptr(k_cache), ptr(v_cache)
    p.kv_indptr, p.kv_indices, p.kv_last_page_len = ptr(kv_indptr), ptr(kv_indices), ptr(kv_last_page_len)
    p.part_o, p.part_lse = ptr(part_o), ptr(part_lse)
    p.B, p.Hq, p.Hkv = B, Hq, Hkv
    p.num_chunks, p.chunk_tokens = num_chunks, chunk_tokens
    p.kv_start, p.chunk_base = kv_start, chunk_base
    p.part_stride = num_chunks + chunk_base if part_stride is None else part_stride
    p.sm_scale = (1.0 / HEAD_DIM ** 0.5) if sm_scale is None else sm_scale
    return p


def decode_partial(p: DecodeParams, G: int, stream=None, variant: int = 0):
    _check(lib().pdattn_decode_partial(ctypes.byref(p), G, variant, stream_ptr(stream)),
           "pdattn_decode_partial")


def merge_states(part_o, part_lse, out, lse, rows: int, num_chunks: int, stream=None):
    _check(lib().pdattn_merge_states(ptr(part_o), ptr(part_lse), ptr(out), ptr(lse), rows,
                                     num_chunks, stream_ptr(stream)), "pdattn_merge_states")


def decode_workspace_size(B: int, Hq: int, part_stride: int) -> int:
    return int(lib().pdattn_decode_workspace_size(B, Hq, part_stride))


def workspace_partials(ws: Workspace, B: int, Hq: int, part_stride: int):
    po, pl = ctypes.c_void_p(), ctypes.c_void_p()
    _check(lib().pdattn_workspace_partials(ctypes.byref(ws), B, Hq, part_stride,
                                           ctypes.byref(po), ctypes.byref(pl)), "pdattn_workspace_partials")
    return po.value, pl.value


def decode_attention(p: DecodeParams, G: int, out, lse, ws: Workspace, stream=None, variant: int = 0):
    _check(lib().pdattn_decode_attention(ctypes.byref(p), G, variant, ptr(out), ptr(lse),
                                         ctypes.byref(ws), stream_ptr(stream)), "pdattn_decode_attention")


NOALLOC_SCRATCH_BYTES = 16 << 20   # PDATTN_NOALLOC_SCRATCH_BYTES


def decode_attention_noalloc(p: DecodeParams, G: int, out, lse, stream=None, variant: int = 0):
    """pdattn_decode_attention_noalloc: decode_attention with the partial states in the library's
    own device array (no allocation, no workspace)."""
    _check(lib().pdattn_decode_attention_noalloc(ctypes.byref(p), G, variant, ptr(out), ptr(lse),
                                                 stream_ptr(stream)), "pdattn_decode_attention_noalloc")


def decode_attention_balanced(p: DecodeParams, G: int, out, lse, ws: Workspace, stream=None,
                              variant: int = 0):
    """pdattn_decode_attention_balanced: decode_attention's arguments, page ranges on the device."""
    _check(lib().pdattn_decode_attention_balanced(ctypes.byref(p), G, variant, ptr(out), ptr(lse),
                                                  ctypes.byref(ws), stream_ptr(stream)),
           "pdattn_decode_attention_balanced")


def decode_balanced_workspace_size(p: DecodeParams, G: int) -> int:
    return int(lib().pdattn_decode_balanced_workspace_size(ctypes.byref(p), G))


def workspace_reserve(ws: Workspace, nbytes: int):
    _check(lib().pdattn_workspace_reserve(ctypes.byref(ws), nbytes), "pdattn_workspace_reserve")


def workspace_release(ws: Workspace):
    lib().pdattn_workspace_release(ctypes.byref(ws))


# ---- balanced path ---------------------------------------------------------------------------

SCHEDULE_SEGMENTS = 24      # PDATTN_SCHEDULE_SEGMENTS
SCHEDULE_WG_INTS = 200      # PDATTN_SCHEDULE_WG_INTS


class Plan:
    """pdattn_plan: balanced schedule of one batch, built from host page-table copies."""

    def __init__(self, kv_indptr, kv_last_page_len, B: int, Hq: int, Hkv: int,
                 force_workgroups: int = 0, chunk_pages: int = 0):
        self._h = ctypes.c_void_p()
        ip, ipp = host_i32(kv_indptr)
        la, lap = host_i32(kv_last_page_len)
        _check(lib().pdattn_plan_create(ipp, lap, B, Hq, Hkv, force_workgroups, chunk_pages,
                                        ctypes.byref(self._h)), "pdattn_plan_create")

    def info(self) -> PlanInfo:
        inf = PlanInfo()
        _check(lib().pdattn_plan_get_info(self._h, ctypes.byref(inf)), "pdattn_plan_get_info")
        return inf

    def schedule(self, with_header: bool = False):
        """(segments, merge_list): segments[w] is a list of 8-int segments
        {b, kvh, qa, npg, t0, t1, jpos, slot}; merge_list is an (n, 4) array {b, kvh, slot0, nc}.
        with_header: also the merge list's header {tag, n_entries, cmax, 0} (cmax > 0: contributor
        k of entry e is slot e * cmax + k)."""
        import numpy as np
        inf = self.info()
        buf = np.zeros(inf.schedule_ints, dtype=np.int32)
        _check(lib().pdattn_plan_get_schedule(self._h, buf.ctypes.data_as(ctypes.c_void_p),
                                              buf.size), "pdattn_plan_get_schedule")
        W = inf.workgroups
        segs = []
        for w in range(W):
            d = buf[w * SCHEDULE_WG_INTS:(w + 1) * SCHEDULE_WG_INTS]
            segs.append([d[8 + 8 * i:16 + 8 * i].tolist() for i in range(int(d[0]))])
        lst = buf[W * SCHEDULE_WG_INTS:].reshape(-1, 4)
        if with_header:
            return segs, lst[1:], lst[0].tolist()
        return segs, lst[1:]

    @property
    def workspace_bytes(self) -> int:
        return int(lib().pdattn_plan_workspace_size(self._h))

    def upload(self, workspace, nbytes: int, stream=None):
        _check(lib().pdattn_plan_upload(self._h, ptr(workspace), nbytes, stream_ptr(stream)),
               "pdattn_plan_upload")

    def run(self, q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, out, lse,
            workspace, nbytes: int, sm_scale=None, stream=None):
        sc = (1.0 / HEAD_DIM ** 0.5) if sm_scale is None else sm_scale
        _check(lib().pdattn_plan_run(self._h, ptr(q), ptr(k_cache), ptr(v_cache), ptr(kv_indptr),
                                     ptr(kv_indices), ptr(kv_last_page_len), ctypes.c_float(sc),
                                     ptr(out), ptr(lse), ptr(workspace), nbytes, stream_ptr(stream)),
               "pdattn_plan_run")

    def run_part(self, parts: int, q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, out,
                 lse, workspace, nbytes: int, sm_scale=None, stream=None):
        """pdattn_plan_run_part: RUN_DECODE, RUN_MERGE or RUN_ALL (for timing each launch)."""
        sc = (1.0 / HEAD_DIM ** 0.5) if sm_scale is None else sm_scale
        _check(lib().pdattn_plan_run_part(self._h, ptr(q), ptr(k_cache), ptr(v_cache), ptr(kv_indptr),
                                          ptr(kv_indices), ptr(kv_last_page_len), ctypes.c_float(sc),
                                          ptr(out), ptr(lse), ptr(workspace), nbytes, stream_ptr(stream),
                                          parts), "pdattn_plan_run_part")

    def close(self):
        if self._h:
            lib().pdattn_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- paged KV append ---------------------------------------------------------------------------

def append_kv(k_new, v_new, k_cache, v_cache, kv_indptr, kv_indices, batch_idx, positions,
              B: int, Hkv: int, n_invalid=None, stream=None):
    """pdattn_append_kv: write token t's K/V rows at position positions[t] of sequence
    batch_idx[t] (the page table already covers the appended tokens)."""
    n = int(batch_idx.shape[0]) if hasattr(batch_idx, "shape") else len(batch_idx)
    _check(lib().pdattn_append_kv(ptr(k_new), ptr(v_new), ptr(k_cache), ptr(v_cache), ptr(kv_indptr),
                                  ptr(kv_indices), ptr(batch_idx), ptr(positions), n, B, Hkv,
                                  ptr(n_invalid) if n_invalid is not None else None,
                                  stream_ptr(stream)), "pdattn_append_kv")


# ---- cascade ---------------------------------------------------------------------------------

def shared_prefix_pages(indptr, indices) -> int:
    ip, ipp = host_i32(indptr)
    ix, ixp = host_i32(indices)
    r = lib().pdattn_shared_prefix_pages(ipp, ixp, len(ip) - 1 if len(indptr) > 0 else 0)
    if r < 0:
        _check(-r, "pdattn_shared_prefix_pages")
    return r


def cascade_prefix(pp: PrefixParams, stream=None):
    _check(lib().pdattn_cascade_prefix(ctypes.byref(pp), stream_ptr(stream)), "pdattn_cascade_prefix")


class CascadePlan:
    """pdattn_cascade_plan (plan_cascade, 01_decode_attention.cu:664-701)."""

    def __init__(self, base: DecodeParams, indptr, indices, lens, d_indices, min_prefix: int = 256,
                 tree: bool = False):
        """tree=False: the reference's single shared prefix; tree=True: a shared-prefix tree
        (pdattn_cascade_tree_plan_create)."""
        self._h = ctypes.c_void_p()
        ip, ipp = host_i32(indptr)
        ix, ixp = host_i32(indices)
        ln, lnp = host_i32(lens)
        fn = lib().pdattn_cascade_tree_plan_create if tree else lib().pdattn_cascade_plan_create
        _check(fn(ctypes.byref(base), ipp, ixp, lnp, ptr(d_indices), min_prefix, ctypes.byref(self._h)),
               "pdattn_cascade_tree_plan_create" if tree else "pdattn_cascade_plan_create")

    def info(self) -> CascadeInfo:
        inf = CascadeInfo()
        _check(lib().pdattn_cascade_plan_get_info(self._h, ctypes.byref(inf)), "pdattn_cascade_plan_get_info")
        return inf

    def decode(self, out, lse, ws: Workspace, stream=None):
        _check(lib().pdattn_cascade_decode(self._h, ptr(out), ptr(lse), ctypes.byref(ws), stream_ptr(stream)),
               "pdattn_cascade_decode")

    def set_mode(self, mode: int):
        """CASCADE_FUSED, CASCADE_SERIAL or CASCADE_TWO_STREAMS (pdattn_cascade_set_mode)."""
        _check(lib().pdattn_cascade_set_mode(self._h, int(mode)), "pdattn_cascade_set_mode")

    def close(self):
        if self._h:
            lib().pdattn_cascade_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- measurement helpers ---------------------------------------------------------------------

def stream_read(buf, nbytes: int, sink, stream=None):
    _check(lib().pdattn_stream_read(ptr(buf), nbytes, ptr(sink), stream_ptr(stream)), "pdattn_stream_read")


def flush_cache(buf, nbytes: int, stream=None):
    _check(lib().pdattn_flush_cache(ptr(buf), nbytes, stream_ptr(stream)), "pdattn_flush_cache")


def device_info() -> DeviceInfo:
    inf = DeviceInfo()
    _check(lib().pdattn_get_device_info(ctypes.byref(inf)), "pdattn_get_device_info")
    return inf
