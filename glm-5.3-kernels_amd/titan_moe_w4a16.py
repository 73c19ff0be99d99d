# SPDX-License-Identifier: Apache-2.0
"""W4A16 group-32 MoE expert GEMMs on MI355X: the step after the small route
aligner (titan_moe_align.titan_moe_align_small) in a GLM-5.3 decode MoE layer.

At the reference's call site (integration/patch_moe_align.py:17-44) the
aligner's sorted_ids / expert_ids / postpad feed vLLM's fused Marlin MoE:
two moe_wna16_marlin_gemm launches around a SiLU-and-multiply with clamp,
then moe_sum (the sequence profiles/sm74/titan_prefill/marlin.py:424-444 runs;
its gate, marlin.py:255-310, fixes the geometry: bf16 activations, E = 288,
top-8, hidden 4096, per-rank intermediate 512 under TP4, uint4b8 codes with
bf16 group-32 scales, no zero points, clamp limit 10, router weight applied
to the output).  This module computes the same layer with two gfx950 kernels
behind glm53_moe_w4a16_gate_up / glm53_moe_w4a16_down; fused_moe_w4a16 runs
the aligner and both in one call.

Weights arrive in the checkpoint's GPTQ / compressed-tensors packing (int32
[E, n_out, K/8], k = 8w + i in bits 4i of word w; bf16 scales [E, n_out,
K/32]) and are repacked once with repack_w4a16 into the kernels' tile order
(the MI355X counterpart of Marlin's load-time repack and scale permutation).
"""
from __future__ import annotations

import math

import torch

import _glm53_lib as _lib

NUM_EXPERTS = 288
TOPK = 8
MAX_TOKENS = 8
GROUP = 32
CLAMP_LIMIT = 10.0


def _check_repacked(w: torch.Tensor, name: str, n_out: int, k: int) -> None:
    want = (w.shape[0], n_out // 16, k // 128, 64, 4)
    if w.dtype != torch.int32 or tuple(w.shape) != want or not w.is_contiguous():
        raise ValueError(f"{name} must be a contiguous repacked int32 tensor of shape {want} "
                         f"(repack_w4a16 output), got {w.dtype} {tuple(w.shape)}")


def _check_scale(s: torch.Tensor, name: str, e: int, n_out: int, k: int) -> None:
    want = (e, n_out // 16, k // 128, 16, 4)
    if s.dtype != torch.bfloat16 or tuple(s.shape) != want or not s.is_contiguous():
        raise ValueError(f"{name} must be contiguous repacked bf16 group-{GROUP} scales of shape {want} "
                         f"(repack_w4a16 output), got {s.dtype} {tuple(s.shape)}")


def _clamp(clamp_limit) -> float:
    if clamp_limit is None:
        return math.inf
    c = float(clamp_limit)
    if not c > 0:
        raise ValueError(f"clamp_limit must be positive or None, got {clamp_limit}")
    return c


def repack_w4a16(weight_packed: torch.Tensor, weight_scale: torch.Tensor):
    """Checkpoint int32 [E, n_out, K/8] codes and bf16 [E, n_out, K/32]
    scales -> the kernels' tile order: (int32 [E, n_out/16, K/128, 64, 4],
    bf16 [E, n_out/16, K/128, 16, 4]); same bytes, reordered (n_out % 16 == 0,
    K % 128 == 0).  Runs once per weight at load time."""
    if weight_packed.dtype != torch.int32 or weight_packed.dim() != 3:
        raise ValueError(f"expected int32 [E, n_out, K/8], got {weight_packed.dtype} {tuple(weight_packed.shape)}")
    e, n_out, kw = weight_packed.shape
    k = 8 * kw
    if n_out % 16 or k % 128 or e == 0:
        raise ValueError(f"n_out ({n_out}) must be a multiple of 16 and K ({k}) of 128")
    if weight_scale.dtype != torch.bfloat16 or tuple(weight_scale.shape) != (e, n_out, k // GROUP):
        raise ValueError(f"expected bf16 scales [{e}, {n_out}, {k // GROUP}], got {weight_scale.dtype} "
                         f"{tuple(weight_scale.shape)}")
    src = weight_packed.contiguous()
    src_s = weight_scale.contiguous()
    out = torch.empty((e, n_out // 16, k // 128, 64, 4), dtype=torch.int32, device=src.device)
    out_s = torch.empty((e, n_out // 16, k // 128, 16, 4), dtype=torch.bfloat16, device=src.device)
    L = _lib.load()
    with torch.cuda.device(src.device):
        rc = L.glm53_moe_w4a16_repack(src.data_ptr(), src_s.data_ptr(), e, n_out, k, out.data_ptr(),
                                      out_s.data_ptr(), _lib.stream_handle(src.device))
    _lib.check(rc, "glm53_moe_w4a16_repack")
    return out, out_s


def moe_w4a16_gate_up(hidden_states: torch.Tensor, w13: torch.Tensor, w13_scale: torch.Tensor,
                      sorted_ids: torch.Tensor, expert_ids: torch.Tensor, topk: int = TOPK,
                      clamp_limit: float | None = CLAMP_LIMIT) -> torch.Tensor:
    """First GEMM + activation over the aligner's blocks: returns c2, bf16
    [T * topk, N], row r = t * topk + j (rows of routes the aligner dropped
    are left unwritten)."""
    T, K = hidden_states.shape
    E = w13.shape[0]
    n2 = w13.shape[1] * 16
    N = n2 // 2
    _check_repacked(w13, "w13", n2, K)
    _check_scale(w13_scale, "w13_scale", E, n2, K)
    if hidden_states.dtype != torch.bfloat16 or hidden_states.stride(1) != 1:
        raise ValueError("hidden_states must be bf16 with contiguous rows")
    R = T * topk
    if sorted_ids.dtype != torch.int32 or expert_ids.dtype != torch.int32 or sorted_ids.numel() < 8 * R \
            or expert_ids.numel() < R:
        raise ValueError("sorted_ids int32 [8*T*topk] and expert_ids int32 [T*topk] expected")
    act = torch.empty((R, N), dtype=torch.bfloat16, device=hidden_states.device)
    L = _lib.load()
    with torch.cuda.device(hidden_states.device):
        rc = L.glm53_moe_w4a16_gate_up(hidden_states.data_ptr(), hidden_states.stride(0), w13.data_ptr(),
                                       w13_scale.data_ptr(), sorted_ids.data_ptr(), expert_ids.data_ptr(),
                                       R, topk, E, N, K, _clamp(clamp_limit), act.data_ptr(),
                                       _lib.stream_handle(hidden_states.device))
    _lib.check(rc, "glm53_moe_w4a16_gate_up")
    return act


def moe_w4a16_down(act: torch.Tensor, w2: torch.Tensor, w2_scale: torch.Tensor, topk_weights: torch.Tensor,
                   topk_ids: torch.Tensor, output: torch.Tensor | None = None) -> torch.Tensor:
    """Second GEMM, router weights and the sum over each token's routes:
    returns bf16 [T, K]."""
    T, topk = topk_ids.shape
    E = w2.shape[0]
    K = w2.shape[1] * 16
    N = act.shape[1]
    _check_repacked(w2, "w2", K, N)
    _check_scale(w2_scale, "w2_scale", E, K, N)
    if act.dtype != torch.bfloat16 or not act.is_contiguous() or act.shape[0] != T * topk:
        raise ValueError("act must be contiguous bf16 [T * topk, N]")
    if topk_weights.dtype != torch.float32 or tuple(topk_weights.shape) != (T, topk):
        raise ValueError("topk_weights must be fp32 [T, topk]")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("topk_ids must be int32 or int64")
    topk_ids = topk_ids if topk_ids.stride(1) == 1 else topk_ids.contiguous()
    topk_weights = topk_weights if topk_weights.stride(1) == 1 else topk_weights.contiguous()
    if output is None:
        output = torch.empty((T, K), dtype=torch.bfloat16, device=act.device)
    elif output.dtype != torch.bfloat16 or tuple(output.shape) != (T, K) or output.stride(1) != 1:
        raise ValueError("output must be bf16 [T, K] with contiguous rows")
    L = _lib.load()
    with torch.cuda.device(act.device):
        rc = L.glm53_moe_w4a16_down(act.data_ptr(), w2.data_ptr(), w2_scale.data_ptr(), topk_ids.data_ptr(),
                                    int(topk_ids.dtype == torch.int64), topk_ids.stride(0),
                                    topk_weights.data_ptr(), topk_weights.stride(0), T, topk, E, N, K,
                                    output.data_ptr(), output.stride(0), _lib.stream_handle(act.device))
    _lib.check(rc, "glm53_moe_w4a16_down")
    return output


def fused_moe_w4a16(hidden_states: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor,
                    w13_scale: torch.Tensor, w2_scale: torch.Tensor, topk_weights: torch.Tensor,
                    topk_ids: torch.Tensor, *, clamp_limit: float | None = CLAMP_LIMIT,
                    global_num_experts: int = -1, expert_map=None,
                    apply_router_weight_on_input: bool = False,
                    output: torch.Tensor | None = None) -> torch.Tensor:
    """The MoE layer for 1..8 decode tokens: aligner, gate/up GEMM + SiLU
    with clamp, down GEMM with router weights, sum over the 8 routes.

    hidden_states bf16 [T, K]; (w13, w13_scale) and (w2, w2_scale) as
    repack_w4a16 returns them for [288, 2N, K/8] / [288, K, N/8] codes with
    [288, 2N, K/32] / [288, K, N/32] bf16 scales; topk_weights fp32 [T, 8];
    topk_ids int32 / int64 [T, 8].
    Returns bf16 [T, K] (written into `output` when given).  Raises
    ValueError outside the configuration the reference's gate accepts
    (profiles/sm74/titan_prefill/marlin.py:255-310): no expert map, router
    weight on the output, 288 experts, top-8, 1..8 tokens."""
    if expert_map is not None:
        raise ValueError("expert_map (expert parallelism) is not supported")
    if apply_router_weight_on_input:
        raise ValueError("the router weight is applied to the output only")
    if hidden_states.dim() != 2 or hidden_states.dtype != torch.bfloat16 or hidden_states.stride(1) != 1:
        raise ValueError("hidden_states must be bf16 [T, K] with contiguous rows")
    T, K = hidden_states.shape
    if not 1 <= T <= MAX_TOKENS:
        raise ValueError(f"1 <= tokens <= {MAX_TOKENS} required, got {T}")
    if topk_ids.dim() != 2 or tuple(topk_ids.shape) != (T, TOPK) or not topk_ids.is_contiguous() \
            or topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"topk_ids must be contiguous int32/int64 [T, {TOPK}]")
    if topk_weights.dtype != torch.float32 or tuple(topk_weights.shape) != (T, TOPK) \
            or not topk_weights.is_contiguous():
        raise ValueError(f"topk_weights must be contiguous fp32 [T, {TOPK}]")
    E = w13.shape[0]
    if E != NUM_EXPERTS or w2.shape[0] != E or global_num_experts not in (-1, E):
        raise ValueError(f"{NUM_EXPERTS} experts required, got {E} (global {global_num_experts})")
    n2 = w13.shape[1] * 16
    N = n2 // 2
    _check_repacked(w13, "w13", n2, K)
    _check_repacked(w2, "w2", K, N)
    _check_scale(w13_scale, "w13_scale", E, n2, K)
    _check_scale(w2_scale, "w2_scale", E, K, N)
    clamp = _clamp(clamp_limit)
    tensors = (hidden_states, w13, w2, w13_scale, w2_scale, topk_weights, topk_ids)
    if not all(t.is_cuda and t.device == hidden_states.device for t in tensors):
        raise ValueError("every tensor must be on the same CUDA (HIP) device")
    if output is None:
        output = torch.empty((T, K), dtype=torch.bfloat16, device=hidden_states.device)
    elif output.dtype != torch.bfloat16 or tuple(output.shape) != (T, K) or output.stride(1) != 1:
        raise ValueError("output must be bf16 [T, K] with contiguous rows")
    L = _lib.load()
    ws_bytes = L.glm53_fused_moe_w4a16_workspace_bytes(T, TOPK, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=hidden_states.device)
    with torch.cuda.device(hidden_states.device):
        rc = L.glm53_fused_moe_w4a16(hidden_states.data_ptr(), hidden_states.stride(0), w13.data_ptr(),
                                     w13_scale.data_ptr(), w2.data_ptr(), w2_scale.data_ptr(),
                                     topk_ids.data_ptr(), int(topk_ids.dtype == torch.int64),
                                     topk_weights.data_ptr(), T, TOPK, E, N, K, clamp,
                                     ws.data_ptr(), ws_bytes, output.data_ptr(), output.stride(0),
                                     _lib.stream_handle(hidden_states.device))
    _lib.check(rc, "glm53_fused_moe_w4a16")
    return output
