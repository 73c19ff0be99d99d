"""Child process of tests/test_zz_no_alloc.py::test_noalloc_first_call_in_graph_capture:
in a fresh process (so the library has not yet looked up the device address
of its static scratch), the first glm53_sparse_mla_noalloc call is made
under HIP graph capture; the graph is replayed twice with different q and
each replay is compared bit for bit with glm53_sparse_mla and a caller
workspace.  Exit status 0 on success."""
import ctypes
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "glm-5.3-kernels_amd")]

import torch  # noqa: E402

import workloads as W  # noqa: E402


def main():
    import _glm53_lib as lib
    from titan_kv import store_int8
    L = lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = W.writer_small(dev, seed=W.SEED_FIXTURE)
    store_int8(w["x"], w["cache"], w["slots"])
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(dev, 91)
    T, H, topk, splits = 8, 16, 2176, 23
    idx = torch.randint(-16, n + 16, (T, 1, topk), generator=g, device=dev, dtype=torch.int32)
    q = torch.empty(T, H, 512, dtype=torch.bfloat16, device=dev)
    out = torch.empty(T, H, 512, dtype=torch.bfloat16, device=dev)
    args = lambda qq: (qq.data_ptr(), qq.stride(0), qq.stride(1), kv.data_ptr(), kv.stride(0), n,
                       idx.data_ptr(), idx.stride(0), T, H, topk, ctypes.c_double(W.SM_SCALE), splits)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    rc = []
    print("[child] capturing the first noalloc call of the process", flush=True)
    with torch.cuda.graph(graph):
        rc.append(L.glm53_sparse_mla_noalloc(*args(q), out.data_ptr(), out.stride(0), out.stride(1),
                                             lib.stream_handle(dev)))
    if rc[0] != 0:
        print(f"[child] noalloc under capture returned {rc[0]}", flush=True)
        return 1
    for r in range(2):
        qr = torch.randn(T, H, 512, generator=g, device=dev).to(torch.bfloat16)
        q.copy_(qr)
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = torch.empty_like(out)
        ws_bytes = L.glm53_sparse_mla_workspace_bytes(T, H, splits)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        lib.check(L.glm53_sparse_mla(*args(qr), ws.data_ptr(), ws_bytes, want.data_ptr(), want.stride(0),
                                     want.stride(1), lib.stream_handle(dev)), "glm53_sparse_mla")
        torch.cuda.synchronize()
        same = torch.equal(got, want)
        print(f"[child] replay {r}: bit-identical to the workspace entry: {same}", flush=True)
        if not same:
            return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
