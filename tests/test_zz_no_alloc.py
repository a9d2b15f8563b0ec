"""fl_decode_attn_dense_noalloc (the allocation-free entry point) against
fl_decode_attn_dense with a caller workspace, through the C ABI: the same kernels and
grid, so outputs and logits are bit-identical.  Two calls in a row on one GPU, the
second over a smaller cache (the static scratch keeps the first call's partials), then
the size limit."""

import ctypes as C

import pytest
import torch

from flashloop_amd import CrossLoopKVLayer, _lib
from flashloop_amd.synthetic import SCALING, decode_workload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(b, h, t, seed):
    w = decode_workload(b, h, t, seed=seed, device=DEV)
    layer = CrossLoopKVLayer.from_prefill([w.keys[r][:, :, :t].contiguous() for r in range(4)],
                                          [w.values[r][:, :, :t].contiguous() for r in range(4)])
    cur = [w.current(r) for r in range(4)]
    return layer, w.queries, cur


def _both(layer, queries, cur, loop, logits):
    lib = _lib.load()
    view = layer.view()
    rows = layer.rows
    q = queries[loop].reshape(rows, 128).contiguous()
    kc = cur[loop][0].reshape(rows, 128).contiguous()
    vc = cur[loop][1].reshape(rows, 128).contiguous()
    cap = layer.logits_capacity()
    stream = torch.cuda.current_stream().cuda_stream
    res = []
    for noalloc in (False, True):
        out = torch.full((rows, 128), float("nan"), dtype=torch.float32, device=DEV)
        lg = torch.full((rows, cap), float("nan"), dtype=torch.float32, device=DEV) if logits else None
        lp = lg.data_ptr() if logits else None
        if noalloc:
            rc = lib.fl_decode_attn_dense_noalloc(C.byref(view), loop, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                                  float(SCALING), out.data_ptr(), lp, cap if logits else 0, stream)
        else:
            nbytes = lib.fl_decode_attn_dense_workspace(C.byref(view))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
            rc = lib.fl_decode_attn_dense(C.byref(view), loop, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                          float(SCALING), out.data_ptr(), lp, cap if logits else 0, ws.data_ptr(),
                                          nbytes, stream)
        _lib.check(rc, "noalloc" if noalloc else "workspace")
        res.append((out, lg))
    torch.cuda.synchronize()
    return res


def test_noalloc_matches_workspace_entry_point():
    print("case: noalloc B4 H8 T6000 then B2 H3 T700", flush=True)
    for (b, h, t, seed) in ((4, 8, 6000, 41), (2, 3, 700, 42)):  # second call smaller
        layer, queries, cur = _case(b, h, t, seed)
        keys = t + 1
        for loop in range(4):
            logits = loop == 1
            (o_ws, l_ws), (o_na, l_na) = _both(layer, queries, cur, loop, logits)
            assert bool(torch.isfinite(o_na).all())
            assert torch.equal(o_ws, o_na), f"B{b} H{h} T{t} loop {loop}: outputs differ"
            if logits:
                assert torch.equal(l_ws[:, :keys], l_na[:, :keys]), f"B{b} H{h} T{t}: logits differ"


def test_noalloc_rejects_caches_beyond_its_scratch():
    print("case: noalloc size limit", flush=True)
    lib = _lib.load()
    assert lib.fl_decode_attn_dense_noalloc_max_bytes() == 8 << 20
    v = _lib.FlCacheView()
    v.batch, v.heads, v.token_capacity, v.tail_capacity = 9000, 1, 64, 128
    need = lib.fl_decode_attn_dense_workspace(C.byref(v))
    assert need > lib.fl_decode_attn_dense_noalloc_max_bytes()
    rc = lib.fl_decode_attn_dense_noalloc(C.byref(v), 0, None, None, None, 1.0, None, None, 0, None)
    assert rc == _lib.FL_E_CAPACITY
    assert b"static scratch" in lib.fl_last_error()
