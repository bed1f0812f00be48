"""PyTorch operators over the C ABI, for use from a serving stack.

``torch.ops.pdattn.paged_decode`` runs the balanced decode path (pdattn_plan_run) and
``torch.ops.pdattn.append_kv`` the paged KV append (pdattn_append_kv); both launch on the
current stream. They are registered with ``torch.library.custom_op``, with fake (shape-only)
implementations, so they trace under torch.compile and work with torch's stream and graph
machinery. The arithmetic is the library's: these functions only pass tensors through.

The balanced plan is built on the host from host copies of kv_indptr and kv_last_page_len
(``indptr_host`` / ``last_host``, int32 CPU tensors), the way FlashInfer's plan() works. Plans and
their workspaces are cached by the contents of those tables, so a decode loop over one batch
composition plans once.
"""
from __future__ import annotations

from collections import OrderedDict

import torch

from . import HEAD_DIM, Plan, append_kv as _append_kv

_PLAN_CACHE_SIZE = 8
_plans: "OrderedDict[tuple, tuple]" = OrderedDict()


def _plan_for(indptr_host: torch.Tensor, last_host: torch.Tensor, Hq: int, Hkv: int,
              device: torch.device):
    ip = indptr_host.to(torch.int32).contiguous()
    la = last_host.to(torch.int32).contiguous()
    key = (ip.numpy().tobytes(), la.numpy().tobytes(), Hq, Hkv, device.index)
    hit = _plans.get(key)
    if hit is not None:
        _plans.move_to_end(key)
        return hit
    B = ip.numel() - 1
    plan = Plan(ip.numpy(), la.numpy(), B, Hq, Hkv)
    ws = torch.empty(max(256, plan.workspace_bytes), dtype=torch.uint8, device=device)
    plan.upload(ws, ws.numel(), torch.cuda.current_stream(device))
    _plans[key] = (plan, ws)
    if len(_plans) > _PLAN_CACHE_SIZE:
        _, (old_plan, _) = _plans.popitem(last=False)
        old_plan.close()
    return plan, ws


@torch.library.custom_op("pdattn::paged_decode", mutates_args=())
def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                 indptr_host: torch.Tensor, last_host: torch.Tensor,
                 sm_scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Paged GQA decode attention. q [B, Hq, 128] fp16; k_cache / v_cache [num_pages, 16, Hkv,
    128] fp16; kv_indptr [B+1], kv_indices [nnz], kv_last_page_len [B] int32 on the device, and
    host copies of kv_indptr / kv_last_page_len. Returns (out [B, Hq, 128] fp16, lse [B, Hq] fp32,
    the natural log of the scaled scores)."""
    if q.dtype != torch.float16 or k_cache.dtype != torch.float16 or v_cache.dtype != torch.float16:
        raise TypeError("q, k_cache and v_cache must be float16")
    if q.dim() != 3 or q.shape[2] != HEAD_DIM or k_cache.dim() != 4 or k_cache.shape[3] != HEAD_DIM:
        raise ValueError("q must be [B, Hq, 128] and the caches [num_pages, 16, Hkv, 128]")
    B, Hq = q.shape[0], q.shape[1]
    Hkv = k_cache.shape[2]
    if indptr_host.numel() != B + 1 or last_host.numel() != B:
        raise ValueError("host page-table copies do not match the batch size")
    q = q.contiguous()
    plan, ws = _plan_for(indptr_host, last_host, Hq, Hkv, q.device)
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=q.device)
    plan.run(q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, out, lse, ws, ws.numel(),
             sm_scale=sm_scale, stream=torch.cuda.current_stream(q.device))
    return out, lse


@paged_decode.register_fake
def _paged_decode_fake(q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, indptr_host,
                       last_host, sm_scale):
    return torch.empty_like(q), q.new_empty((q.shape[0], q.shape[1]), dtype=torch.float32)


@torch.library.custom_op("pdattn::append_kv", mutates_args=("k_cache", "v_cache"))
def append_kv(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
              v_cache: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
              batch_idx: torch.Tensor, positions: torch.Tensor) -> None:
    """Write k_new / v_new [n, Hkv, 128] fp16 into the paged caches at (batch_idx[t],
    positions[t]); the page table already covers the appended tokens."""
    if k_new.dtype != torch.float16 or k_cache.dtype != torch.float16:
        raise TypeError("K/V rows and caches must be float16")
    B = kv_indptr.numel() - 1
    _append_kv(k_new.contiguous(), v_new.contiguous(), k_cache, v_cache, kv_indptr, kv_indices,
               batch_idx, positions, B, k_cache.shape[2],
               stream=torch.cuda.current_stream(k_cache.device))


@append_kv.register_fake
def _append_kv_fake(k_new, v_new, k_cache, v_cache, kv_indptr, kv_indices, batch_idx, positions):
    return None
