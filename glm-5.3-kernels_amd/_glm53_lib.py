"""ctypes binding of libglm53_hip.so (the C ABI declared in include/glm53.h).

Loading the library does not touch the GPU.  If the library is missing the
import fails loudly: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libglm53_hip.so"
ABI_VERSION = 3

EXPORTED = (
    "glm53_abi_version",
    "glm53_error_string",
    "glm53_store_int8",
    "glm53_sparse_mla_workspace_bytes",
    "glm53_sparse_mla",
    "glm53_sparse_mla_noalloc",
    "glm53_convert_req_index",
    "glm53_sparse_mla_paged",
    "glm53_expand_pools",
    "glm53_sparse_mla_pooled",
    "glm53_sparse_mla_partials_bytes",
    "glm53_sparse_mla_partials",
    "glm53_sparse_mla_merge",
    "glm53_sparse_mla_gather_floor",
    "glm53_moe_align_small",
    "glm53_moe_w4a16_repack",
    "glm53_moe_w4a16_gate_up",
    "glm53_moe_w4a16_down",
    "glm53_fused_moe_w4a16_workspace_bytes",
    "glm53_fused_moe_w4a16",
    "glm53_fp8_paged_mqa_logits",
    "glm53_indexer_topk_workspace_bytes",
    "glm53_indexer_topk",
    "glm53_stream_probe",
)

_lib = None


def load():
    """Return the loaded library, raising if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build the HIP kernels first "
            "(python glm-5.3-kernels_amd/build_lib.py or __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB_PATH))
    P, I64, I, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
    L.glm53_abi_version.restype = I
    L.glm53_abi_version.argtypes = []
    L.glm53_error_string.restype = ctypes.c_char_p
    L.glm53_error_string.argtypes = [I]
    L.glm53_store_int8.restype = I
    L.glm53_store_int8.argtypes = [P, I64, P, I64, I64, I64, I64, P, I, I64, P]
    L.glm53_sparse_mla_workspace_bytes.restype = I64
    L.glm53_sparse_mla_workspace_bytes.argtypes = [I64, I64, I64]
    L.glm53_sparse_mla.restype = I
    L.glm53_sparse_mla.argtypes = [P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, D, I64, P, I64,
                                   P, I64, I64, P]
    L.glm53_sparse_mla_noalloc.restype = I
    L.glm53_sparse_mla_noalloc.argtypes = [P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, D, I64,
                                           P, I64, I64, P]
    L.glm53_convert_req_index.restype = I
    L.glm53_convert_req_index.argtypes = [P, P, I64, I64, I64, P, I64, P, I64, I64, I64, I64, I64, P]
    L.glm53_sparse_mla_paged.restype = I
    L.glm53_sparse_mla_paged.argtypes = [P, I64, I64, P, I64, I64, I64, P, I64, P, P, I64, I64, I64, I64,
                                         I64, I64, I64, D, I64, P, I64, P, I64, I64, P]
    L.glm53_expand_pools.restype = I
    L.glm53_expand_pools.argtypes = [P, I, I64, I64, P, I64, P, I64, I64, I64, P]
    L.glm53_sparse_mla_pooled.restype = I
    L.glm53_sparse_mla_pooled.argtypes = [P, I64, I64, P, I64, I64, I64, P, I64, I64, P, I64, P, P, I64, I64,
                                          I64, I64, I64, I64, I64, D, I64, P, I64, P, I64, I64, P]
    L.glm53_sparse_mla_partials_bytes.restype = I64
    L.glm53_sparse_mla_partials_bytes.argtypes = [I64, I64, I64]
    L.glm53_sparse_mla_partials.restype = I
    L.glm53_sparse_mla_partials.argtypes = [P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, D, I64, P,
                                            I64, P]
    L.glm53_sparse_mla_merge.restype = I
    L.glm53_sparse_mla_merge.argtypes = [P, I64, I64, I64, I64, P, I64, I64, P]
    L.glm53_sparse_mla_gather_floor.restype = I
    L.glm53_sparse_mla_gather_floor.argtypes = [P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, I64, P, I64, P]
    L.glm53_moe_align_small.restype = I
    L.glm53_moe_align_small.argtypes = [P, I, I64, P, P, P, P]
    F = ctypes.c_float
    L.glm53_moe_w4a16_repack.restype = I
    L.glm53_moe_w4a16_repack.argtypes = [P, P, I64, I64, I64, P, P, P]
    L.glm53_moe_w4a16_gate_up.restype = I
    L.glm53_moe_w4a16_gate_up.argtypes = [P, I64, P, P, P, P, I64, I64, I64, I64, I64, F, P, P]
    L.glm53_moe_w4a16_down.restype = I
    L.glm53_moe_w4a16_down.argtypes = [P, P, P, P, I, I64, P, I64, I64, I64, I64, I64, I64, P, I64, P]
    L.glm53_fused_moe_w4a16_workspace_bytes.restype = I64
    L.glm53_fused_moe_w4a16_workspace_bytes.argtypes = [I64, I64, I64]
    L.glm53_fused_moe_w4a16.restype = I
    L.glm53_fused_moe_w4a16.argtypes = [P, I64, P, P, P, P, P, I, P, I64, I64, I64, I64, I64, F, P, I64,
                                        P, I64, P]
    L.glm53_fp8_paged_mqa_logits.restype = I
    L.glm53_fp8_paged_mqa_logits.argtypes = [P, I64, I64, P, I64, I64, I64, P, I64, P, P, I64, I64, I64, I64,
                                             I64, I64, I, P, I64, P]
    L.glm53_indexer_topk_workspace_bytes.restype = I64
    L.glm53_indexer_topk_workspace_bytes.argtypes = [I64, I64, I64]
    L.glm53_indexer_topk.restype = I
    L.glm53_indexer_topk.argtypes = [P, I64, P, I64, I64, I64, P, I64, P, I64, P]
    L.glm53_stream_probe.restype = I
    L.glm53_stream_probe.argtypes = [I, P, P, I64, P]
    version = L.glm53_abi_version()
    if version != ABI_VERSION:
        raise ImportError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}")
    _lib = L
    return L


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().glm53_error_string(rc).decode(errors="replace")
        raise RuntimeError(f"{what} failed: {msg} (code {rc})")


def stream_handle(device) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream
