"""Torch-tensor front end of the C ABI: argument checks, output allocation, streams.

Each function launches on torch's current HIP stream and returns torch tensors.  The
names follow the reference wrappers they replace (flashloop/kivi_backend.py:678-992,
flashloop/engine.py:346-498, flashloop/prefill.py:158-237).
"""

from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib
from ._lib import GROUP, HEAD_DIM, check, load, ptr_array


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require(t: torch.Tensor, dtype, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _vec(t: torch.Tensor, rows: int, name: str) -> torch.Tensor:
    """[B,H,1,128] / [B,H,128] / [B*H,128] bf16 -> contiguous [B*H,128]."""
    t = t.reshape(rows, HEAD_DIM)
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16")
    return t.contiguous()


# ---------------------------------------------------------------------------- J1
def pack_kv_groups(view, loops, src_keys, src_values, *, src_bh_stride, src_row_offset, dst_group0, n_groups,
                   masks=(None, None), mask_stride=0, recon_keys=None, recon_values=None) -> None:
    """Encode 64-token groups of ``src_*`` (bf16 ``[B*H, rows, 128]`` views) into ``view``."""
    lib = load()
    keys = ptr_array([t.data_ptr() for t in src_keys] + [0] * (4 - len(src_keys)))
    vals = ptr_array([t.data_ptr() for t in src_values] + [0] * (4 - len(src_values)))
    m = ptr_array([_p(x) or 0 for x in masks])
    rk = ptr_array([_p(x) or 0 for x in recon_keys] + [0] * (4 - len(recon_keys))) if recon_keys else None
    rv = ptr_array([_p(x) or 0 for x in recon_values] + [0] * (4 - len(recon_values))) if recon_values else None
    rc = lib.fl_pack_kv_groups(
        C.byref(view), loops, C.cast(keys, _lib._PP), C.cast(vals, _lib._PP), src_bh_stride, src_row_offset,
        C.cast(m, _lib._PP), mask_stride, dst_group0.data_ptr(), n_groups,
        C.cast(rk, _lib._PP) if rk is not None else None, C.cast(rv, _lib._PP) if rv is not None else None,
        _stream(),
    )
    check(rc, "fl_pack_kv_groups")


# ---------------------------------------------------------------------------- J2
class Workspace:
    """Grow-only device scratch reused across calls ordered on one stream (the reference
    keeps per-layer split-KV workspaces the same way, flashloop/cache.py:672-704)."""

    def __init__(self) -> None:
        self._buf: torch.Tensor | None = None

    def get(self, nbytes: int, device) -> torch.Tensor:
        if self._buf is None or self._buf.numel() < nbytes or self._buf.device != torch.device(device):
            self._buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        return self._buf


_WS = Workspace()


def fused_dense_pair(view, queries, keys, values, scaling, *, logits_capacity, device,
                     workspace: Workspace | None = None):
    """Loops 1 and 2 of a decode step in one reader launch (``fl_decode_attn_dense_pair``).
    Returns (out loop 1 f32 [B*H,128], out loop 2, loop-2 logits f32 [B*H, logits_capacity])."""
    lib = load()
    rows = view.batch * view.heads
    qs = [_vec(x, rows, "query") for x in queries]
    ks = [_vec(x, rows, "current_key") for x in keys]
    vs = [_vec(x, rows, "current_value") for x in values]
    out0 = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    out1 = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    logits = torch.empty(rows, logits_capacity, dtype=torch.float32, device=device)
    ws_bytes = lib.fl_decode_attn_dense_pair_workspace(C.byref(view))
    ws = (workspace or _WS).get(ws_bytes, device)
    rc = lib.fl_decode_attn_dense_pair(
        C.byref(view), qs[0].data_ptr(), ks[0].data_ptr(), vs[0].data_ptr(), out0.data_ptr(),
        qs[1].data_ptr(), ks[1].data_ptr(), vs[1].data_ptr(), out1.data_ptr(), float(scaling),
        logits.data_ptr(), logits.shape[1], ws.data_ptr(), ws.numel(), _stream(),
    )
    check(rc, "fl_decode_attn_dense_pair")
    return out0, out1, logits


def fused_dense_source_attention(view, loop, query, current_key, current_value, scaling, *, return_logits,
                                 logits_capacity, device, workspace: Workspace | None = None, out=None, logits=None):
    """``dense_source_attention_cuda`` replacement.  Returns (out f32 [B*H,128], logits or None)."""
    lib = load()
    rows = view.batch * view.heads
    q = _vec(query, rows, "query")
    kc = _vec(current_key, rows, "current_key")
    vc = _vec(current_value, rows, "current_value")
    if out is None:
        out = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    if return_logits and logits is None:
        logits = torch.empty(rows, logits_capacity, dtype=torch.float32, device=device)
    ws_bytes = lib.fl_decode_attn_dense_workspace(C.byref(view))
    ws = (workspace or _WS).get(ws_bytes, device)
    rc = lib.fl_decode_attn_dense(
        C.byref(view), loop, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), float(scaling), out.data_ptr(),
        _p(logits) if return_logits else None, logits.shape[1] if return_logits else 0,
        ws.data_ptr(), ws.numel(), _stream(),
    )
    check(rc, "fl_decode_attn_dense")
    return out, (logits if return_logits else None)


SELECT_MAX_STRIDE = 35 * 1024  # logits rows the register-resident top-k holds
SELECT_MAX_KEYS = 8 * 1024     # selections its LDS list holds


def dense_select_fits(logits_capacity: int, fraction: float) -> bool:
    """Whether ``fused_dense_select`` takes rows of this stride at this fraction."""
    return 0 < logits_capacity <= SELECT_MAX_STRIDE and math.ceil(logits_capacity * fraction) <= SELECT_MAX_KEYS


def fused_dense_select(view, loop, query, current_key, current_value, scaling, fraction, capacity, *,
                       logits_capacity, device, workspace: Workspace | None = None):
    """Dense read of loop ``loop`` with logits, then the top-k of those logits and the merge
    of the read's rows in one launch (``fl_decode_attn_dense_select``): the results of
    ``fused_dense_source_attention(..., return_logits=True)`` followed by
    ``decode_topk`` on each row's ``packed + tail + 1`` keys, two launches instead of three
    (plus the key-count arithmetic).  Returns (out, logits, indices, valid, mass, weights,
    counts)."""
    lib = load()
    rows = view.batch * view.heads
    q = _vec(query, rows, "query")
    kc = _vec(current_key, rows, "current_key")
    vc = _vec(current_value, rows, "current_value")
    out = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    logits = torch.empty(rows, logits_capacity, dtype=torch.float32, device=device)
    idx = torch.empty(rows, capacity, dtype=torch.int32, device=device)
    valid = torch.empty(rows, capacity, dtype=torch.uint8, device=device)
    mass = torch.empty(rows, dtype=torch.float32, device=device)
    w = torch.empty(rows, capacity, dtype=torch.float32, device=device)
    counts = torch.empty(rows, dtype=torch.int32, device=device)
    ws_bytes = lib.fl_decode_attn_dense_workspace(C.byref(view))
    ws = (workspace or _WS).get(ws_bytes, device)
    rc = lib.fl_decode_attn_dense_select(
        C.byref(view), loop, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), float(scaling), out.data_ptr(),
        logits.data_ptr(), logits.shape[1], float(fraction), capacity, idx.data_ptr(), valid.data_ptr(),
        mass.data_ptr(), w.data_ptr(), counts.data_ptr(), None, ws.data_ptr(), ws.numel(), _stream(),
    )
    check(rc, "fl_decode_attn_dense_select")
    return out, logits, idx, valid, mass, w, counts


def decode_capacity(keys: int, fraction: float) -> int:
    """Budget and padded capacity (flashloop/engine.py:443-452, 84-109)."""
    k = min(keys, max(1, math.ceil(keys * fraction)))
    return (k // GROUP + 1) * GROUP


def decode_topk(logits: torch.Tensor, n_keys: torch.Tensor, fraction: float, capacity: int,
                rows_per_count: int = 1, validate: bool = False, nonfinite: torch.Tensor | None = None):
    """Top-k of each logits row by fp32 softmax weight (ties to the lower index) ->
    (indices i32, valid u8, mass f32, weights f32, counts i32).

    ``nonfinite`` (optional i32 [rows]) receives each row's count of NaN/inf scores.
    ``validate=True`` waits for the kernel and raises ``ValueError`` when a row holds one
    (as ``flashloop/selection.py:78-79`` refuses non-finite decode weights); the engine
    path leaves it off, like the reference engine (``flashloop/engine.py:438-453``)."""
    _require(logits, torch.float32, "logits")
    _require(n_keys, torch.int32, "n_keys")
    rows = logits.shape[0]
    dev = logits.device
    idx = torch.empty(rows, capacity, dtype=torch.int32, device=dev)
    valid = torch.empty(rows, capacity, dtype=torch.uint8, device=dev)
    mass = torch.empty(rows, dtype=torch.float32, device=dev)
    w = torch.empty(rows, capacity, dtype=torch.float32, device=dev)
    counts = torch.empty(rows, dtype=torch.int32, device=dev)
    if validate and nonfinite is None:
        nonfinite = torch.empty(rows, dtype=torch.int32, device=dev)
    if nonfinite is not None:
        _require(nonfinite, torch.int32, "nonfinite")
        if nonfinite.numel() < rows:
            raise ValueError("nonfinite needs one entry per row")
    rc = load().fl_decode_topk(logits.data_ptr(), logits.stride(0), rows, n_keys.data_ptr(), rows_per_count,
                               float(fraction), capacity, idx.data_ptr(), valid.data_ptr(), mass.data_ptr(),
                               w.data_ptr(), counts.data_ptr(), nonfinite.data_ptr() if nonfinite is not None else None,
                               _stream())
    check(rc, "fl_decode_topk")
    if validate:
        bad = int((nonfinite[:rows] != 0).sum().item())
        if bad:
            raise ValueError(f"decode top-k: {bad} score row(s) hold NaN or infinite values")
    return idx, valid, mass, w, counts


def _counts_ptr(counts, rows):
    """Device pointer of the optional per-row selected counts (i32 [rows]) or None."""
    if counts is None:
        return None
    counts = counts.reshape(rows)
    _require(counts, torch.int32, "counts")
    return counts.data_ptr()


def fused_cross_loop_pv(view, loop, indices, valid, weights, current_value, *, device,
                        workspace: Workspace | None = None, counts=None):
    """``pv_cross_loop_cuda`` + current-token term replacement (engine.py:346-371).
    ``counts``: optional i32 ``[B*H]`` selected slots per row (every valid slot of row r
    lies below counts[r], as the top-k writes them): the reader then skips the padding."""
    lib = load()
    rows = view.batch * view.heads
    cap = indices.shape[-1]
    indices = indices.reshape(rows, cap)
    valid = valid.reshape(rows, cap)
    weights = weights.reshape(rows, cap)
    _require(indices, torch.int32, "indices")
    _require(valid, torch.uint8, "valid")
    _require(weights, torch.float32, "weights")
    vc = _vec(current_value, rows, "current_value")
    out = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    ws = (workspace or _WS).get(lib.fl_decode_selected_workspace(C.byref(view), cap), device)
    rc = lib.fl_decode_selected_pv(C.byref(view), loop, indices.data_ptr(), valid.data_ptr(), weights.data_ptr(),
                                   cap, _counts_ptr(counts, rows), vc.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                   ws.numel(), _stream())
    check(rc, "fl_decode_selected_pv")
    return out


def fused_sparse_attention_delta(view, loop, query, current_key, current_value, indices, valid,
                                 source_selected_output, global_mass, scaling, *, device,
                                 workspace: Workspace | None = None, counts=None):
    """``sparse_attention_delta_cuda`` replacement -> delta f32 [B*H,128] (``counts`` as
    in ``fused_cross_loop_pv``)."""
    lib = load()
    rows = view.batch * view.heads
    cap = indices.shape[-1]
    indices = indices.reshape(rows, cap)
    valid = valid.reshape(rows, cap)
    _require(indices, torch.int32, "indices")
    _require(valid, torch.uint8, "valid")
    src = source_selected_output.reshape(rows, HEAD_DIM).float().contiguous()
    mass = global_mass.reshape(rows).float().contiguous()
    q = _vec(query, rows, "query")
    kc = _vec(current_key, rows, "current_key")
    vc = _vec(current_value, rows, "current_value")
    out = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    ws = (workspace or _WS).get(lib.fl_decode_selected_workspace(C.byref(view), cap), device)
    rc = lib.fl_decode_attn_sparse_delta(C.byref(view), loop, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                         indices.data_ptr(), valid.data_ptr(), cap, _counts_ptr(counts, rows),
                                         src.data_ptr(),
                                         mass.data_ptr(), float(scaling), out.data_ptr(), ws.data_ptr(),
                                         ws.numel(), _stream())
    check(rc, "fl_decode_attn_sparse_delta")
    return out


def fused_sparse_attention_delta_with_source(view, loop, query, current_key, current_value, indices, valid,
                                             source_weights, source_current_value, global_mass, scaling, *,
                                             device, workspace: Workspace | None = None, counts=None):
    """Loop-3/4 cached-mass delta that also forms the loop-2 selected aggregate from the
    rows it reads.  Returns (delta f32 [B*H,128], source_output f32 [B*H,128])
    (``counts`` as in ``fused_cross_loop_pv``)."""
    lib = load()
    rows = view.batch * view.heads
    cap = indices.shape[-1]
    indices = indices.reshape(rows, cap)
    valid = valid.reshape(rows, cap)
    weights = source_weights.reshape(rows, cap)
    _require(indices, torch.int32, "indices")
    _require(valid, torch.uint8, "valid")
    _require(weights, torch.float32, "source_weights")
    mass = global_mass.reshape(rows).float().contiguous()
    q = _vec(query, rows, "query")
    kc = _vec(current_key, rows, "current_key")
    vc = _vec(current_value, rows, "current_value")
    vc1 = _vec(source_current_value, rows, "source_current_value")
    out = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    src = torch.empty(rows, HEAD_DIM, dtype=torch.float32, device=device)
    ws = (workspace or _WS).get(lib.fl_decode_selected_workspace(C.byref(view), cap), device)
    rc = lib.fl_decode_attn_sparse_delta_fused(C.byref(view), loop, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                               indices.data_ptr(), valid.data_ptr(), weights.data_ptr(),
                                               vc1.data_ptr(), cap, _counts_ptr(counts, rows), mass.data_ptr(),
                                               float(scaling),
                                               src.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    check(rc, "fl_decode_attn_sparse_delta_fused")
    return out, src


# ---------------------------------------------------------------------------- J4
def _rows_view(t: torch.Tensor, dim: int):
    """(outer, rows, row_bytes, outer_stride_bytes, row_stride_bytes) of ``t`` seen as
    [prod(shape[:dim]), shape[dim], prod(shape[dim+1:])]."""
    if not t.is_contiguous():
        raise ValueError("row movement needs contiguous tensors")
    es = t.element_size()
    outer = 1
    for s in t.shape[:dim]:
        outer *= s
    inner = 1
    for s in t.shape[dim + 1:]:
        inner *= s
    rows = t.shape[dim]
    return outer, rows, inner * es, rows * inner * es, inner * es


def gather_rows(src: torch.Tensor, index: torch.Tensor, dim: int) -> torch.Tensor:
    """``src.index_select(dim, index)`` on the device (flashloop/prefill.py:158)."""
    _require(index, torch.int32, "index")
    shape = list(src.shape)
    shape[dim] = index.numel()
    dst = torch.empty(shape, dtype=src.dtype, device=src.device)
    o, rows, rb, so, sr = _rows_view(src, dim)
    _, _, _, do, dr = _rows_view(dst, dim)
    err = torch.zeros(1, dtype=torch.int32, device=src.device)
    rc = load().fl_gather_rows(src.data_ptr(), so, sr, rows, dst.data_ptr(), do, dr, o, rb, index.data_ptr(),
                               index.numel(), err.data_ptr(), _stream())
    check(rc, "fl_gather_rows")
    return dst, err


def scatter_rows_(dst: torch.Tensor, index: torch.Tensor, src: torch.Tensor, dim: int):
    """``dst.index_copy_(dim, index, src)`` on the device (flashloop/prefill.py:193-194, 237)."""
    _require(index, torch.int32, "index")
    if src.dtype != dst.dtype:
        raise ValueError("src and dst dtypes differ")
    o, rows, rb, do, dr = _rows_view(dst, dim)
    o2, n, rb2, so, sr = _rows_view(src, dim)
    if o2 != o or rb2 != rb or n != index.numel():
        raise ValueError("src shape does not match dst/index")
    err = torch.zeros(1, dtype=torch.int32, device=dst.device)
    rc = load().fl_scatter_rows(src.data_ptr(), so, sr, dst.data_ptr(), do, dr, rows, o, rb, index.data_ptr(),
                                index.numel(), err.data_ptr(), _stream())
    check(rc, "fl_scatter_rows")
    return dst, err


def hidden_delta_score(current: torch.Tensor, previous: torch.Tensor) -> torch.Tensor:
    """``_hidden_delta_score`` (flashloop/engine.py:78-81) for bf16 ``[..., dim]`` rows."""
    if current.shape != previous.shape:
        raise ValueError("hidden shapes differ")
    cur = current.contiguous()
    prev = previous.contiguous()
    _require(cur, torch.bfloat16, "current")
    _require(prev, torch.bfloat16, "previous")
    dim = cur.shape[-1]
    rows = cur.numel() // dim
    out = torch.empty(cur.shape[:-1], dtype=torch.float32, device=cur.device)
    check(load().fl_hidden_delta_score(cur.data_ptr(), prev.data_ptr(), rows, dim, out.data_ptr(), _stream()),
          "fl_hidden_delta_score")
    return out


def select_tokens(scores: torch.Tensor, fraction: float, eligible: torch.Tensor | None = None,
                  force_last_token: bool = True):
    """``select_prefill_tokens`` (flashloop/selection.py:26-69) -> (mask bool, positions, counts, err)."""
    scores = scores.float().contiguous()
    b, t = scores.shape
    el = None
    if eligible is not None:
        if eligible.shape != scores.shape:
            raise ValueError("eligible must match scores")
        el = eligible.to(torch.uint8).contiguous()
    mask = torch.empty(b, t, dtype=torch.uint8, device=scores.device)
    pos = torch.empty(b, t, dtype=torch.int32, device=scores.device)
    counts = torch.empty(b, dtype=torch.int32, device=scores.device)
    err = torch.zeros(1, dtype=torch.int32, device=scores.device)
    rc = load().fl_select_tokens(scores.data_ptr(), b, t, float(fraction), _p(el), int(bool(force_last_token)),
                                 mask.data_ptr(), pos.data_ptr(), counts.data_ptr(), err.data_ptr(), _stream())
    check(rc, "fl_select_tokens")
    return mask.bool(), pos, counts, err


# ---------------------------------------------------------------------------- decode-step model ops
EPI_PLAIN, EPI_F32, EPI_ADD, EPI_SWIGLU, EPI_ROPE = range(5)


def _rows2d(x: torch.Tensor, name: str) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"{name} must be bf16 or f32")
    if not x2.is_cuda:
        raise RuntimeError(f"{name} must be a device tensor")
    return x2.contiguous()


def gemv(x: torch.Tensor, weights, *, epilogue: int = EPI_PLAIN, addend: torch.Tensor | None = None,
         rope: tuple[torch.Tensor, torch.Tensor] | None = None, head_dim: int = HEAD_DIM):
    """``x @ W.T`` for the M <= 8 rows of a decode step (``fl_gemv_bf16``).  ``x``: [..., K]
    bf16 or f32 (f32 is rounded to bf16 first); ``weights``: list of [N, K] bf16.  Returns
    [M, N] (bf16, f32 for EPI_F32), or (q, k, v) for EPI_ROPE."""
    x2 = _rows2d(x, "x")
    m, k = x2.shape
    ws = [w if w.is_contiguous() else w.contiguous() for w in weights]
    for w in ws:
        _require(w, torch.bfloat16, "weight")
    n = ws[0].shape[0]
    dt = torch.float32 if epilogue == EPI_F32 else torch.bfloat16
    nout = 3 if epilogue == EPI_ROPE else 1
    outs = [torch.empty(m, n, dtype=dt, device=x2.device) for _ in range(nout)]
    add = None
    if epilogue == EPI_ADD:
        add = addend.reshape(m, n)
        _require(add, torch.bfloat16, "addend")
    cos = sin = None
    if epilogue == EPI_ROPE:
        cos, sin = (t.reshape(m, head_dim).contiguous() for t in rope)
        _require(cos, torch.bfloat16, "rope cos")
        _require(sin, torch.bfloat16, "rope sin")
    rc = load().fl_gemv_bf16(
        x2.data_ptr(), int(x2.dtype == torch.float32), k, m, k, C.cast(ptr_array([w.data_ptr() for w in ws]), _lib._PP),
        n, int(epilogue), C.cast(ptr_array([o.data_ptr() for o in outs]), _lib._PP), n, _p(add), n,
        _p(cos), _p(sin), int(head_dim), _stream(),
    )
    check(rc, "fl_gemv_bf16")
    return tuple(outs) if epilogue == EPI_ROPE else outs[0]


def norm_chain(r: torch.Tensor, *, x: torch.Tensor | None = None, w_a: torch.Tensor | None = None,
               w_f: torch.Tensor | None = None, w_b: torch.Tensor | None = None, eps: float,
               want_h: bool = True):
    """``h = r + RMSNorm_a(x)`` (or ``h = r``), then optionally ``h = RMSNorm_f(h)``, and
    ``z = RMSNorm_b(h)`` (``fl_norm_chain``).  Returns (h or None, z or None), [M, D] bf16."""
    r2 = _rows2d(r, "r")
    m, d = r2.shape
    x2 = None if x is None else _rows2d(x, "x")
    for t, nm in ((r2, "r"), (x2, "x")):
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError(f"{nm} must be bf16")
    h = torch.empty(m, d, dtype=torch.bfloat16, device=r2.device) if want_h else None
    z = torch.empty(m, d, dtype=torch.bfloat16, device=r2.device) if w_b is not None else None
    rc = load().fl_norm_chain(m, d, float(eps), _p(x2), r2.data_ptr(), _p(w_a), _p(w_f), _p(w_b), _p(h), _p(z), d,
                              _stream())
    check(rc, "fl_norm_chain")
    return h, z


def gemv_chain(r: torch.Tensor, weights, *, x: torch.Tensor | None = None, w_a: torch.Tensor | None = None,
               w_f: torch.Tensor | None = None, w_b: torch.Tensor | None = None, eps: float, want_h: bool = True,
               epilogue: int = EPI_PLAIN, addend: torch.Tensor | None = None,
               rope: tuple[torch.Tensor, torch.Tensor] | None = None, head_dim: int = HEAD_DIM):
    """``norm_chain`` followed by ``gemv`` of its output (z, or h without ``w_b``) in one
    launch (``fl_gemv_bf16_chain``), bit-identical to the two calls.  Returns (h or None,
    the GEMV output as ``gemv`` returns it)."""
    r2 = _rows2d(r, "r")
    m, d = r2.shape
    x2 = None if x is None else _rows2d(x, "x")
    for t, nm in ((r2, "r"), (x2, "x")):
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError(f"{nm} must be bf16")
    ws = [w if w.is_contiguous() else w.contiguous() for w in weights]
    for w in ws:
        _require(w, torch.bfloat16, "weight")
    n = ws[0].shape[0]
    dt = torch.float32 if epilogue == EPI_F32 else torch.bfloat16
    nout = 3 if epilogue == EPI_ROPE else 1
    outs = [torch.empty(m, n, dtype=dt, device=r2.device) for _ in range(nout)]
    add = None
    if epilogue == EPI_ADD:
        add = addend.reshape(m, n)
        _require(add, torch.bfloat16, "addend")
    cos = sin = None
    if epilogue == EPI_ROPE:
        cos, sin = (t.reshape(m, head_dim).contiguous() for t in rope)
        _require(cos, torch.bfloat16, "rope cos")
        _require(sin, torch.bfloat16, "rope sin")
    h = torch.empty(m, d, dtype=torch.bfloat16, device=r2.device) if want_h else None
    rc = load().fl_gemv_bf16_chain(
        m, d, float(eps), _p(x2), r2.data_ptr(), _p(w_a), _p(w_f), _p(w_b), _p(h), d,
        C.cast(ptr_array([w.data_ptr() for w in ws]), _lib._PP), n, int(epilogue),
        C.cast(ptr_array([o.data_ptr() for o in outs]), _lib._PP), n, _p(add), n, _p(cos), _p(sin), int(head_dim),
        _stream(),
    )
    check(rc, "fl_gemv_bf16_chain")
    return h, (tuple(outs) if epilogue == EPI_ROPE else outs[0])


def append_tail(view, keys, values, tail_active, tail_tokens: torch.Tensor) -> None:
    """Device half of a decode append (``fl_append_tail``): rows ``keys[r]``/``values[r]``
    ([B, H, 1, 128] bf16, r = loop) to each sequence's tail at its device length."""
    rows = view.batch * view.heads
    ks = [_vec(k, rows, "key") for k in keys]
    vs = [_vec(v, rows, "value") for v in values]
    for t in tail_active:
        _require(t, torch.uint8, "tail_active")
    _require(tail_tokens, torch.int32, "tail_tokens")
    rc = load().fl_append_tail(
        C.byref(view), C.cast(ptr_array([k.data_ptr() for k in ks]), _lib._PP),
        C.cast(ptr_array([v.data_ptr() for v in vs]), _lib._PP),
        C.cast(ptr_array([t.data_ptr() for t in tail_active]), _lib._PP), tail_tokens.data_ptr(), _stream(),
    )
    check(rc, "fl_append_tail")
