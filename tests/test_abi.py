"""The C ABI boundary (include/pdattn.h) -- CPU only, no compute calls.

Checks that libpdattn.so loads, exports every function the header declares, and that the
host-only entry points (planning, validation, prefix detection, sizes) behave as documented
without touching a GPU.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
import pdattn
from pdattn import inputs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pdattn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pdattn_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 20
    lib = pdattn.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(pdattn.EXPORTS) == names


def test_strerror_names_every_status():
    for code, name in pdattn.STATUS.items():
        assert pdattn.lib().pdattn_strerror(code).decode() == name
    assert pdattn.lib().pdattn_strerror(99).decode() == "PDATTN_ERR_UNKNOWN"


def test_params_struct_matches_reference_field_order():
    """pdattn_decode_params keeps DecodeParams' fields in order (01_decode_attention.cu:51-65)."""
    names = [f[0] for f in pdattn.DecodeParams._fields_]
    assert names == ["q", "k_cache", "v_cache", "kv_indptr", "kv_indices", "kv_last_page_len",
                     "part_o", "part_lse", "B", "Hq", "Hkv", "num_chunks", "chunk_tokens",
                     "kv_start", "chunk_base", "part_stride", "sm_scale"]
    assert ctypes.sizeof(pdattn.DecodeParams) == 8 * 8 + 9 * 4 + 4  # 8 pointers, 9 x 32-bit, padding


def test_shared_prefix_pages_matches_oracle():
    rng = np.random.default_rng(0)
    for _ in range(200):
        B = int(rng.integers(0, 6))
        shared = list(rng.integers(0, 8, size=int(rng.integers(0, 6))))
        indptr, indices = [0], []
        for b in range(B):
            seq = shared + list(rng.integers(0, 8, size=int(rng.integers(0, 4))))
            indices += seq
            indptr.append(len(indices))
        assert pdattn.shared_prefix_pages(indptr, indices) == oracle.shared_prefix_pages(indptr, indices)
    sp = inputs.make_shared_prefix_batch(8192, [512] * 64, 32, 8, seed=21, fill=False)
    assert pdattn.shared_prefix_pages(sp.indptr, sp.indices) == 512


def test_shared_prefix_rejects_bad_table():
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.shared_prefix_pages([0, 3, 2], [1, 2, 3])
    assert e.value.status == 3


@pytest.mark.parametrize("max_len,force", [(1, 1), (17, 1), (4097, 7), (32768, 13), (0, 1), (1000, 64)])
def test_plan_chunks_forced_invariants(max_len, force):
    nc, ct = pdattn.plan_chunks(4, 1, 8, max_len, force)
    assert ct % 16 == 0 and ct >= 16
    assert nc >= 1 and nc <= max(force, 1)
    assert nc * ct >= max_len
    assert (nc - 1) * ct < max(max_len, 1)


def test_plan_chunks_rejects_bad_group():
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.plan_chunks(3, 1, 8, 100, 1)
    assert e.value.status == 2


def test_decode_workspace_size():
    assert pdattn.decode_workspace_size(2, 32, 7) >= 2 * 32 * 7 * 129 * 4
    assert pdattn.decode_workspace_size(0, 32, 7) == 0


def _params(B=1, Hq=32, Hkv=8, **kw):
    fake = 1 << 20  # aligned stand-in address; validation fails before any device access
    return pdattn.make_params(fake, fake, fake, fake, fake, fake, B, Hq, Hkv, **kw)


@pytest.mark.parametrize("kw,status", [
    (dict(Hq=24, Hkv=8), 2),               # G = 3
    (dict(Hq=30, Hkv=8), 2),               # Hq % Hkv != 0
    (dict(num_chunks=0), 1),
    (dict(num_chunks=4, part_stride=3), 1),
    (dict(kv_start=-1), 1),
])
def test_decode_partial_validation(kw, status):
    p = _params(**{k: v for k, v in kw.items() if k in ("Hq", "Hkv")},
                **{k: v for k, v in kw.items() if k not in ("Hq", "Hkv")})
    G = max(1, p.Hq // p.Hkv)
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.decode_partial(p, G if p.Hq % p.Hkv == 0 and G in (1, 2, 4, 8) else 4)
    assert e.value.status == status


def test_decode_attention_rejects_chunk_base():
    p = _params(num_chunks=2, chunk_base=1, part_stride=3)
    ws = pdattn.Workspace()
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.decode_attention(p, 4, 1 << 20, 1 << 20, ws)
    assert e.value.status == 1


def test_caller_workspace_is_never_reallocated():
    ws = pdattn.Workspace(1 << 20, 64, 0)  # caller-provided, too small
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.workspace_reserve(ws, 1 << 16)
    assert e.value.status == 4
    assert ws.base == 1 << 20 and ws.bytes == 64


def test_plan_create_rejects_bad_tables():
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.Plan([0, 4, 2], [16, 16], 2, 32, 8, force_workgroups=4)
    assert e.value.status == 3
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.Plan([0, 4, 6], [16, 0], 2, 32, 8, force_workgroups=4)   # last page empty
    assert e.value.status == 3
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.Plan([0, 4, 6], [16, 17], 2, 32, 8, force_workgroups=4)
    assert e.value.status == 3


def test_plan_run_requires_upload():
    bt = inputs.make_batch([100], 32, 8, seed=1, fill=False)
    plan = pdattn.Plan(bt.indptr, bt.last, 1, 32, 8, force_workgroups=3)
    with pytest.raises(pdattn.PdattnError) as e:
        plan.run(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 30)
    assert e.value.status == 6


def test_check_page_table():
    """pdattn_check_page_table: each malformed table is rejected with PDATTN_ERR_PAGE_TABLE."""
    good = ([0, 2, 2, 5], [4, 0, 3, 1, 2], [7, 0, 16])
    pdattn.check_page_table(*good, num_pages=5)
    pdattn.check_page_table([0], [], [], num_pages=0)   # no sequences
    bad = [
        (([0, 2, 1, 5], [4, 0, 3, 1, 2], [7, 0, 16]), 5, "indptr decreases"),
        (([-1, 2, 2, 5], [4, 0, 3, 1, 2, 0], [7, 0, 16]), 5, "negative indptr"),
        (([0, 2, 2, 5], [4, 0, 3, 5, 2], [7, 0, 16]), 5, "page id == num_pages"),
        (([0, 2, 2, 5], [4, -1, 3, 1, 2], [7, 0, 16]), 5, "negative page id"),
        (([0, 2, 2, 5], [4, 0, 3, 1, 2], [0, 0, 16]), 5, "last page length 0"),
        (([0, 2, 2, 5], [4, 0, 3, 1, 2], [7, 0, 17]), 5, "last page length 17"),
        (([0, 2, 2, 5], [4, 0, 3, 1, 2], [7, 0, 16]), 4, "page id beyond a smaller cache"),
    ]
    for (ip, ix, la), n, what in bad:
        with pytest.raises(pdattn.PdattnError) as e:
            pdattn.check_page_table(ip, ix, la, num_pages=n)
        assert e.value.status == 3, what
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.check_page_table(*good, num_pages=-1)
    assert e.value.status == 1


def test_noalloc_rejects_partials_beyond_its_array():
    """pdattn_decode_attention_noalloc refuses, before any GPU call, a request whose partial states
    exceed PDATTN_NOALLOC_SCRATCH_BYTES; a single chunk needs no partial states."""
    B, Hq, chunks = 64, 32, 256   # 64 * 32 * 256 slots * 516 B = 270 MB
    assert pdattn.decode_workspace_size(B, Hq, chunks) > pdattn.NOALLOC_SCRATCH_BYTES
    p = _params(B=B, Hq=Hq, Hkv=8, num_chunks=chunks, chunk_tokens=16)
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.decode_attention_noalloc(p, 4, 1 << 20, 1 << 20)
    assert e.value.status == 4
    p = _params(num_chunks=2, chunk_base=1, part_stride=3)
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.decode_attention_noalloc(p, 4, 1 << 20, 1 << 20)
    assert e.value.status == 1


@pytest.mark.parametrize("chunk_tokens", [0, 17, 8208])
def test_cascade_prefix_rejects_chunk_sizes(chunk_tokens):
    """Prefix chunks are whole pages, at most 8192 tokens (512 page ids staged per workgroup);
    the check comes before any device work."""
    pp = pdattn.PrefixParams()
    pp.q = pp.k_cache = pp.v_cache = pp.prefix_pages = pp.part_o = pp.part_lse = 1 << 20
    pp.B, pp.Hq, pp.Hkv = 2, 32, 8
    pp.prefix_len, pp.chunk_tokens, pp.part_stride = 16384, chunk_tokens, 1024
    pp.sm_scale = 0.088
    with pytest.raises(pdattn.PdattnError) as e:
        pdattn.cascade_prefix(pp)
    assert e.value.status == 2   # PDATTN_ERR_UNSUPPORTED
