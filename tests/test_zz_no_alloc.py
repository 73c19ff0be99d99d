"""glm53_sparse_mla_noalloc (static device scratch, no allocation) through
the C ABI, against glm53_sparse_mla with a caller workspace: bit-identical
outputs on two calls in a row (the second smaller, reading partial rows the
first left behind in the shared scratch), the single-pass path, and the
size limit rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import workloads as W
from conftest import log_case

pytestmark = pytest.mark.gpu

ERR_SCRATCH_LIMIT = -6
MAX_ROWS = 8192


def _args(q, kv, idx, splits):
    n = kv.shape[0]
    return (q.data_ptr(), q.stride(0), q.stride(1), kv.data_ptr(), kv.stride(0), n,
            idx.data_ptr(), idx.stride(0), q.shape[0], q.shape[1], idx.shape[-1],
            ctypes.c_double(W.SM_SCALE), splits)


def with_workspace(L, lib, q, kv, idx, splits):
    out = torch.empty(q.shape[0], q.shape[1], 512, dtype=torch.bfloat16, device=q.device)
    ws_bytes = L.glm53_sparse_mla_workspace_bytes(q.shape[0], q.shape[1], splits)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    rc = L.glm53_sparse_mla(*_args(q, kv, idx, splits), ws.data_ptr() if ws_bytes else None, ws_bytes,
                            out.data_ptr(), out.stride(0), out.stride(1), lib.stream_handle(q.device))
    lib.check(rc, "glm53_sparse_mla")
    return out


def no_alloc(L, q, kv, idx, splits, out, stream):
    return L.glm53_sparse_mla_noalloc(*_args(q, kv, idx, splits), out.data_ptr(), out.stride(0),
                                      out.stride(1), stream)


def test_noalloc_equals_workspace_entry(cuda):
    import _glm53_lib as lib
    from titan_kv import store_int8
    L = lib.load()
    w = W.writer_small(cuda, seed=W.SEED_FIXTURE)
    store_int8(w["x"], w["cache"], w["slots"])
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 77)
    stream = lib.stream_handle(cuda)
    cases = ((8, 16, 2176, 17, "B=8 x 17 splits: 2176 partial rows"),
             (2, 20, 1024, 8, "B=2, 20 heads x 8 splits: 512 partial rows (smaller, after the larger)"),
             (8, 16, 2176, 23, "B=8 x 23 splits of three tiles (three key groups): 2944 partial rows"),
             (1, 16, 2176, 68, "B=1 x 68 one-tile splits (one key group): 1088 partial rows"),
             (1, 16, 2176, 1, "single pass: no scratch"),
             (4, 64, 2048, 32, "exactly the limit: 4 x 32 x 64 = 8192 partial rows"))
    for T, H, topk, splits, tag in cases:
        q = torch.randn(T, H, 512, generator=g, device=cuda).to(torch.bfloat16)
        idx = torch.randint(-16, n + 16, (T, 1, topk), generator=g, device=cuda, dtype=torch.int32)
        log_case("noalloc", tag)
        want = with_workspace(L, lib, q, kv, idx, splits)
        got = torch.full_like(want, float("nan"))
        rc = no_alloc(L, q, kv, idx, splits, got, stream)
        lib.check(rc, "glm53_sparse_mla_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, want), tag
    # one row past the limit: rejected, nothing launched, out untouched
    T, H, topk, splits = 4, 64, 2048, 33
    assert T * splits * H > MAX_ROWS
    q = torch.randn(T, H, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(0, n, (T, 1, topk), generator=g, device=cuda, dtype=torch.int32)
    sentinel = torch.full((T, H, 512), 3.0, dtype=torch.bfloat16, device=cuda)
    log_case("noalloc over the limit")
    assert no_alloc(L, q, kv, idx, splits, sentinel, stream) == ERR_SCRATCH_LIMIT
    torch.cuda.synchronize()
    assert bool((sentinel == 3.0).all())
    assert b"static scratch" in L.glm53_error_string(ERR_SCRATCH_LIMIT)


def test_noalloc_first_call_in_graph_capture(cuda):
    """The library looks up the device address of its static scratch on the
    first glm53_sparse_mla_noalloc call on a device; made under HIP graph
    capture (in a fresh child process, so that no earlier call did the
    lookup), that call must capture correctly: two replays with different q,
    each bit-identical to glm53_sparse_mla with a caller workspace."""
    import subprocess
    import sys
    from pathlib import Path
    child = Path(__file__).resolve().parent / "noalloc_capture_child.py"
    log_case("noalloc first call under capture (child process)")
    res = subprocess.run([sys.executable, "-u", str(child)], capture_output=True, text=True, timeout=240)
    print(res.stdout, res.stderr[-2000:], flush=True)
    assert res.returncode == 0, res.stdout + res.stderr[-2000:]
