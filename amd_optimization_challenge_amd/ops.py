"""torch-facing wrappers of the C ABI.  PyTorch supplies device memory and the
current HIP stream; every computation runs in libmla_mi355x.so.

All functions take device tensors and enqueue work on
``torch.cuda.current_stream()``; none synchronizes the host.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

QK_DIM = 576
V_DIM = 512
FP4_ROW = 288
MX_BLOCKS = 18


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("tensors must live on a HIP device")


def kv_mode_id(kv_mode) -> int:
    if isinstance(kv_mode, int):
        return kv_mode
    try:
        return _lib.KV_MODES[kv_mode]
    except KeyError:
        raise ValueError(f"unknown kv_mode {kv_mode!r}; expected one of {sorted(_lib.KV_MODES)}")


def as_bytes(t: torch.Tensor) -> torch.Tensor:
    """Reinterpret a 1-byte-element tensor (fp8 / fp4x2 / e8m0 / uint8) as uint8."""
    if t.element_size() != 1:
        raise ValueError(f"expected a 1-byte dtype, got {t.dtype}")
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def cu_count() -> int:
    n = ctypes.c_int(0)
    _lib.check(_lib.load().mla_device_cu_count(ctypes.byref(n)), "mla_device_cu_count")
    return n.value


def workspace_bytes(batch: int, num_heads: int, kv_mode) -> int:
    n = ctypes.c_int64(0)
    _lib.check(_lib.load().mla_workspace_bytes(batch, num_heads, kv_mode_id(kv_mode), ctypes.byref(n)),
               "mla_workspace_bytes")
    return n.value


_ws_cache: dict = {}


def workspace(batch: int, num_heads: int, kv_mode, device) -> torch.Tensor:
    """Workspace for a shape, cached per (shape, device) -- keyed on shapes only."""
    device = torch.device(device)
    key = (batch, num_heads, kv_mode_id(kv_mode), device)
    ws = _ws_cache.get(key)
    if ws is None:
        with torch.cuda.device(device):
            ws = torch.empty(workspace_bytes(batch, num_heads, kv_mode), dtype=torch.uint8, device=device)
        _ws_cache[key] = ws
    return ws


# ---------------------------------------------------------------------------
# quantizers (bit exact to the reference's; see oracle/mla_oracle.py)
# ---------------------------------------------------------------------------


def quant_fp8_per_tensor(x: torch.Tensor, out: torch.Tensor | None = None,
                         scale: torch.Tensor | None = None):
    """bf16 tensor -> (float8_e4m3fn tensor of the same shape, f32 scale [1]).

    competitor_submissions/mi355x_reference/reference.py:65-80 (quantize_fp8).
    """
    _require_cuda(x)
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bfloat16")
    x = x.contiguous()
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    if scale is None:
        scale = torch.empty(1, dtype=torch.float32, device=x.device)
    scratch = torch.empty(8192, dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().mla_quant_fp8_per_tensor(_ptr(x), x.numel(), _ptr(out), _ptr(scale),
                                                        _ptr(scratch), scratch.numel(), _stream()),
                   "mla_quant_fp8_per_tensor")
    return out, scale


def pack_mxfp4(x: torch.Tensor, scale_cols: int | None = None):
    """bf16 [..., cols] -> (packed uint8 [..., cols/2], e8m0 uint8 [rows, scale_cols]).

    competitor_submissions/mi355x_reference/reference.py:88-113 (quantize_mxfp4).
    ``scale_cols`` (>= cols/32) pads the scale rows like AITER may; padding
    bytes are left as 127 (2^0).
    """
    _require_cuda(x)
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bfloat16")
    cols = x.shape[-1]
    if cols % 32:
        raise ValueError("last dim must be a multiple of 32")
    x2 = x.reshape(-1, cols).contiguous()
    rows = x2.shape[0]
    nsc = cols // 32 if scale_cols is None else int(scale_cols)
    if nsc < cols // 32:
        raise ValueError("scale_cols < cols/32")
    packed = torch.empty((rows, cols // 2), dtype=torch.uint8, device=x.device)
    scales = torch.full((rows, nsc), 127, dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().mla_pack_mxfp4(_ptr(x2), rows, cols, x2.stride(0) * 2, _ptr(packed),
                                              packed.stride(0), _ptr(scales), scales.stride(0), _stream()),
                   "mla_pack_mxfp4")
    return packed.reshape(*x.shape[:-1], cols // 2), scales


def append_kv(x: torch.Tensor, slots: torch.Tensor | None, fp8=None, mxfp4=None,
              amax: torch.Tensor | None = None) -> None:
    """Write bf16 tokens ``x`` [n, 576] (or [n, 1, 576]) into cache rows ``slots``.

    ``fp8`` = (cache [rows, 1, 576] e4m3fn, scale [1] f32): quantized with the
    cache's existing scale, the bytes quantize_fp8
    (competitor_submissions/mi355x_reference/reference.py:65-80) gives for the
    whole buffer at that scale.  ``mxfp4`` = (cache [rows, 1, 288] fp4x2,
    e8m0 [rows, >= 18]): the row's dynamic_mxfp4_quant bytes (reference.py:88-113).
    ``slots`` int32 [n] (None = rows 0..n-1, negative = skip).  ``amax``
    (int32 [1], optional) is max-ed with the bf16 bits of max|x|.  The slots
    are trusted to be in range and distinct, like the decode's kv_indices.
    """
    if fp8 is None and mxfp4 is None:
        raise ValueError("append_kv needs an fp8 and/or an mxfp4 cache")
    _require_cuda(x, slots, amax)
    if x.dtype != torch.bfloat16 or x.shape[-1] != QK_DIM:
        raise ValueError("x must be bfloat16 [..., 576]")
    x2 = x.reshape(-1, QK_DIM)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    n = x2.shape[0]
    if slots is not None:
        if slots.dtype != torch.int32 or slots.numel() != n:
            raise ValueError("slots must be int32 with one entry per token")
        slots = slots.contiguous()
    if amax is not None and (amax.dtype != torch.int32 or amax.numel() < 1):
        raise ValueError("amax must be an int32 tensor of >= 1 element")
    f8 = f8_scale = f4 = f4_scales = None
    f8_stride = f4_stride = f4_scale_stride = 0
    if fp8 is not None:
        cache, f8_scale = fp8
        f8 = as_bytes(cache).reshape(cache.shape[0], -1)
        f8_stride = f8.stride(0)
        _require_cuda(f8, f8_scale)
    if mxfp4 is not None:
        cache, sc = mxfp4
        f4 = as_bytes(cache).reshape(cache.shape[0], -1)
        f4_scales = as_bytes(sc)
        f4_stride, f4_scale_stride = f4.stride(0), f4_scales.stride(0)
        _require_cuda(f4, f4_scales)
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().mla_append_kv(_ptr(x2), n, x2.stride(0) * 2, _ptr(slots), _ptr(f8), f8_stride,
                                             _ptr(f8_scale), _ptr(f4), f4_stride, _ptr(f4_scales),
                                             f4_scale_stride, _ptr(amax), _stream()),
                   "mla_append_kv")


# ---------------------------------------------------------------------------
# decode pipeline stages
# ---------------------------------------------------------------------------


def _rows(x: torch.Tensor) -> torch.Tensor:
    """The cache as [rows, bytes per row]: every leading dimension (tokens, or
    pages x page_size x kv heads of a paged cache) flattened into rows."""
    x = x.view(torch.uint8) if x.dtype == torch.bfloat16 else as_bytes(x)
    return x if x.dim() == 2 else x.flatten(0, x.dim() - 2)


def _kv_args(kv_mode: int, kv_data: dict):
    """(k_cache, k_row_stride, k_scales, k_scale_stride, v_cache, v_row_stride, kv_scale)."""
    if kv_mode == 0:
        fp8, sc = kv_data["fp8"]
        k = _rows(fp8)
        return k, k.stride(0), None, 0, None, 0, sc
    if kv_mode == 1:
        fp4, e8 = kv_data["mxfp4"]
        k = _rows(fp4)
        s = _rows(e8)
        return k, k.stride(0), s, s.stride(0), None, 0, None
    if kv_mode == 2:
        fp4, e8 = kv_data["mxfp4"]
        fp8, sc = kv_data["fp8"]
        k = _rows(fp4)
        s = _rows(e8)
        v = _rows(fp8)
        return k, k.stride(0), s, s.stride(0), v, v.stride(0), sc
    if kv_mode == 3:
        k = _rows(kv_data["bf16"])
        if kv_data["bf16"].dtype != torch.bfloat16:
            raise ValueError("kv_data['bf16'] must be a bf16 tensor")
        return k, k.stride(0), None, 0, None, 0, None
    raise ValueError(kv_mode)


def expand_pages(page_indptr: torch.Tensor, page_ids: torch.Tensor, last_page_lens: torch.Tensor,
                 page_size: int):
    """AITER's page table -> the token-level (kv_indptr, kv_indices) over the
    cache viewed as [pages * page_size, row] (``mla_expand_pages``).
    kv_indices has room for every page full; entries past kv_indptr[-1] are
    not written."""
    _require_cuda(page_indptr, page_ids, last_page_lens)
    for name, t in (("page_indptr", page_indptr), ("page_ids", page_ids), ("last_page_lens", last_page_lens)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 tensor")
    batch = page_indptr.numel() - 1
    if batch < 1 or last_page_lens.numel() != batch:
        raise ValueError("page_indptr needs batch + 1 entries and last_page_lens batch entries")
    page_size = int(page_size)
    max_pages = page_ids.numel()
    kv_indptr = torch.empty(batch + 1, dtype=torch.int32, device=page_indptr.device)
    kv_indices = torch.empty(max(max_pages * page_size, 1), dtype=torch.int32, device=page_indptr.device)
    with torch.cuda.device(page_indptr.device):
        _lib.check(_lib.load().mla_expand_pages(
            _ptr(page_indptr), _ptr(page_ids), _ptr(last_page_lens), batch, page_size, max_pages,
            _ptr(kv_indptr), _ptr(kv_indices), _stream()), "mla_expand_pages")
    return kv_indptr, kv_indices


def plan(kv_indptr: torch.Tensor, batch: int, num_heads: int, kv_mode, ws: torch.Tensor,
         q_seq_len: int = 1) -> None:
    """``batch`` = query rows (sequences x q_seq_len)."""
    with torch.cuda.device(ws.device):
        _lib.check(_lib.load().mla_plan(_ptr(kv_indptr), batch, int(q_seq_len), num_heads, kv_mode_id(kv_mode),
                                        _ptr(ws), ws.numel(), _stream()), "mla_plan")


def decode(q_fp8, q_scale, kv_data, kv_indptr, kv_indices, num_heads, sm_scale, kv_mode, ws, out, lse=None):
    """One decode launch over the plan in ``ws``; rows = q_fp8.shape[0]."""
    mode = kv_mode_id(kv_mode)
    k, ks, ksc, kss, v, vs, sc = _kv_args(mode, kv_data)
    batch = q_fp8.shape[0]
    with torch.cuda.device(ws.device):
        _lib.check(_lib.load().mla_decode(
            _ptr(q_fp8), _ptr(q_scale), _ptr(k), ks, _ptr(ksc), kss, _ptr(v), vs, _ptr(sc),
            _ptr(kv_indptr), _ptr(kv_indices), batch, num_heads, float(sm_scale), mode, _ptr(ws),
            ws.numel(), _ptr(out), _ptr(lse), _stream()), "mla_decode")


def combine(batch: int, num_heads: int, ws: torch.Tensor, out: torch.Tensor, lse=None) -> None:
    with torch.cuda.device(ws.device):
        _lib.check(_lib.load().mla_combine(batch, num_heads, _ptr(ws), ws.numel(), _ptr(out), _ptr(lse),
                                           _stream()), "mla_combine")


def decode_fwd(q, kv_data, kv_indptr, kv_indices, sm_scale, kv_mode="fp8", out=None, ws=None, q_seq_len=1,
               return_lse=False, page_size=1, kv_last_page_lens=None, q_dtype="fp8", lse=None):
    """Whole operator: FP8-quantize q, plan, decode, combine.

    q: bf16 [rows, H, 576], rows = sequences x q_seq_len (row i of a sequence
    attends causally to its first L - (q_seq_len - 1 - i) keys).  Returns the
    bf16 [rows, H, 512] output, plus the f32 [rows, H] natural-log lse when
    ``return_lse``.  page_size > 1: a paged cache as AITER's mla_decode_fwd
    takes it (caches [pages, page_size, 1, row], kv_indptr over pages,
    kv_indices = page ids, kv_last_page_lens), expanded on the device first.
    q_dtype "bf16": the a16w8 route (``mla_decode_fwd_a16w8``; 16 heads, fp8
    cache): Q keeps its own precision, no per-tensor quantization.  q_dtype
    "fp8_row" (``mla_decode_fwd_rowq``; 16 heads, fp8 or mxfp4 cache): Q
    quantized per head row inside the decode, which for up to 256 query rows
    also plans its own work (two launches per call).  ``out`` (bf16 [rows, H,
    512]) and ``lse`` (f32 [rows, H], with ``return_lse``) may be passed in;
    each is allocated here only when it is not.
    """
    if int(page_size) != 1:
        if kv_indices is None or kv_last_page_lens is None:
            raise ValueError("a paged cache needs kv_indices (page ids) and kv_last_page_lens")
        kv_indptr, kv_indices = expand_pages(kv_indptr, kv_indices, kv_last_page_lens, page_size)
    _require_cuda(q, kv_indptr, kv_indices)
    if q.dtype != torch.bfloat16 or q.dim() != 3 or q.shape[-1] != QK_DIM:
        raise ValueError("q must be bf16 [rows, heads, 576]")
    if kv_indptr.dtype != torch.int32 or (kv_indices is not None and kv_indices.dtype != torch.int32):
        raise ValueError("kv_indptr / kv_indices must be int32")
    q = q.contiguous()
    batch, num_heads = q.shape[0], q.shape[1]
    q_seq_len = int(q_seq_len)
    if q_seq_len < 1 or batch % q_seq_len != 0 or kv_indptr.numel() != batch // q_seq_len + 1:
        raise ValueError(f"{batch} query rows, q_seq_len {q_seq_len} and {kv_indptr.numel()} kv_indptr "
                         f"entries do not fit (need rows = sequences x q_seq_len, indptr = sequences + 1)")
    mode = kv_mode_id(kv_mode)
    k, ks, ksc, kss, v, vs, sc = _kv_args(mode, kv_data)
    if ws is None:
        ws = workspace(batch, num_heads, mode, q.device)
    if out is None:
        out = torch.empty((batch, num_heads, V_DIM), dtype=torch.bfloat16, device=q.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (batch, num_heads, V_DIM) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bf16 [{batch}, {num_heads}, {V_DIM}] tensor")
    if not return_lse:
        lse = None
    elif lse is None:
        lse = torch.empty((batch, num_heads), dtype=torch.float32, device=q.device)
    elif lse.dtype != torch.float32 or tuple(lse.shape) != (batch, num_heads) or not lse.is_contiguous():
        raise ValueError(f"lse must be a contiguous f32 [{batch}, {num_heads}] tensor")
    routes = {"fp8": "mla_decode_fwd", "bf16": "mla_decode_fwd_a16w8", "fp8_row": "mla_decode_fwd_rowq"}
    if q_dtype not in routes:
        raise ValueError(f"q_dtype must be 'fp8' (a8w8: per-tensor Q quant), 'bf16' (a16w8) or 'fp8_row' "
                         f"(per-row Q quant), got {q_dtype!r}")
    name = routes[q_dtype]
    fn = getattr(_lib.load(), name)
    with torch.cuda.device(q.device):
        _lib.check(fn(
            _ptr(q), _ptr(k), ks, _ptr(ksc), kss, _ptr(v), vs, _ptr(sc), _ptr(kv_indptr),
            _ptr(kv_indices), batch, q_seq_len, num_heads, float(sm_scale), mode, _ptr(ws), ws.numel(),
            _ptr(out), _ptr(lse), _stream()), name)
    return (out, lse) if return_lse else out


def decode_fwd_noalloc(q, kv_data, kv_indptr, kv_indices, sm_scale, kv_mode="fp8", out=None, q_seq_len=1,
                       return_lse=False):
    """``decode_fwd`` through ``mla_decode_fwd_noalloc``: the library's own
    per-device scratch array replaces the workspace, so nothing but ``out``
    (and the lse, when asked for) is allocated here -- pass ``out`` to allocate
    nothing.  Calls that overlap on one device race on that array."""
    _require_cuda(q, kv_indptr, kv_indices, out)
    if q.dtype != torch.bfloat16 or q.dim() != 3 or q.shape[-1] != QK_DIM or not q.is_contiguous():
        raise ValueError("q must be contiguous bf16 [rows, heads, 576]")
    batch, num_heads = q.shape[0], q.shape[1]
    q_seq_len = int(q_seq_len)
    if q_seq_len < 1 or batch % q_seq_len != 0 or kv_indptr.numel() != batch // q_seq_len + 1:
        raise ValueError("query rows, q_seq_len and kv_indptr do not fit")
    mode = kv_mode_id(kv_mode)
    k, ks, ksc, kss, v, vs, sc = _kv_args(mode, kv_data)
    if out is None:
        out = torch.empty((batch, num_heads, V_DIM), dtype=torch.bfloat16, device=q.device)
    lse = torch.empty((batch, num_heads), dtype=torch.float32, device=q.device) if return_lse else None
    with torch.cuda.device(q.device):
        _lib.check(_lib.load().mla_decode_fwd_noalloc(
            _ptr(q), _ptr(k), ks, _ptr(ksc), kss, _ptr(v), vs, _ptr(sc), _ptr(kv_indptr), _ptr(kv_indices),
            batch, q_seq_len, num_heads, float(sm_scale), mode, _ptr(out), _ptr(lse), _stream()),
            "mla_decode_fwd_noalloc")
    return (out, lse) if return_lse else out


def selftest(which: int, inp: torch.Tensor, out: torch.Tensor) -> None:
    with torch.cuda.device(inp.device):
        _lib.check(_lib.load().mla_selftest(which, _ptr(inp), _ptr(out), _stream()), "mla_selftest")


# ---------------------------------------------------------------------------
# workspace introspection (mirrors workspace_layout() in csrc/abi.hip)
# ---------------------------------------------------------------------------
PLAN_HEADER = 16
QUANT_SCRATCH = 8192


def _a256(x: int) -> int:
    return (x + 255) & ~255


def blocks_per_cu(num_heads: int, kv_mode: int) -> int:
    """Resident decode work-groups per CU: 2 for H = 16 with one cache (fp8 or
    mxfp4), else 1; kv_mode < 0 gives the largest over the modes."""
    if num_heads != 16:
        return 1
    return 2 if kv_mode <= 1 else 1


def target_items(batch: int, num_heads: int, kv_mode: int, num_cu: int) -> int:
    """Work items the planner aims for (csrc/abi.hip target_items_for)."""
    slots = num_cu * blocks_per_cu(num_heads, kv_mode)
    if batch < slots:
        return slots
    return min(max(batch, slots * 3 // 2), 4 * slots)


PLAN_MIN_CHUNK = 128


def plan_target(batch: int, num_heads: int, kv_mode: int, num_cu: int, contiguous: bool = False) -> tuple:
    """(items, min_chunk, max_splits) the planner aims for (csrc/abi.hip
    plan_target_for): ``mla_plan`` and the indexed caches use ``target_items``,
    a 128-token chunk floor and no split cap; the fused entry points on a
    contiguous 16-head cache (no kv_indices) aim for one item per CU below
    that many sequences, a 1024-token chunk floor from there up, and at most
    32 pieces per sequence."""
    items, min_chunk, max_splits = target_items(batch, num_heads, kv_mode, num_cu), PLAN_MIN_CHUNK, 0
    if contiguous and num_heads == 16:
        if batch < num_cu:
            items = min(items, num_cu)
        else:
            min_chunk = 1024
        max_splits = 32
    return items, min_chunk, max_splits


def workspace_layout(batch: int, num_heads: int, kv_mode, num_cu: int) -> dict:
    """Byte offsets of the workspace regions; ``total`` equals mla_workspace_bytes.
    Sized for the largest target over the kv modes (``target_items``);
    ``plan_target`` is the one the planner uses for ``kv_mode``."""
    mode = kv_mode_id(kv_mode)
    target = target_items(batch, num_heads, -1, num_cu)
    max_items = target + batch
    off = 0
    lay = {"quant": off}
    off = _a256(off + QUANT_SCRATCH)
    lay["q_fp8"] = off
    off = _a256(off + batch * num_heads * QK_DIM)
    lay["plan"] = off
    off = _a256(off + (PLAN_HEADER + 4 * max_items + 2 * batch) * 4)
    lay["part_o"] = off
    off = _a256(off + max_items * num_heads * V_DIM * 2)  # bf16 split outputs
    lay["part_lse"] = off
    off = _a256(off + max_items * num_heads * 4)
    lay.update(total=off, max_items=max_items, target_items=target,
               plan_target=target_items(batch, num_heads, mode, num_cu))
    return lay


def read_plan(ws: torch.Tensor, batch: int, num_heads: int, kv_mode) -> dict:
    """Copy the device plan back to the host (synchronizes; for tests and tooling)."""
    lay = workspace_layout(batch, num_heads, kv_mode, cu_count())
    mi = lay["max_items"]
    n_words = PLAN_HEADER + 4 * mi + 2 * batch
    words = ws[lay["plan"]: lay["plan"] + 4 * n_words].view(torch.int32).cpu()
    hdr = words[:PLAN_HEADER]
    n = int(hdr[0])
    items = words[PLAN_HEADER: PLAN_HEADER + 4 * mi].reshape(mi, 4)[:n]
    binfo = words[PLAN_HEADER + 4 * mi: PLAN_HEADER + 4 * mi + 2 * batch].reshape(batch, 2)
    return {"num_items": n, "chunk": int(hdr[1]), "total": int(hdr[2]), "batch": int(hdr[3]),
            "max_items": int(hdr[4]), "items": items, "batch_info": binfo, "layout": lay}
