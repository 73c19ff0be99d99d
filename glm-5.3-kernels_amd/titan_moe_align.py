# SPDX-License-Identifier: Apache-2.0
"""Single-workgroup stable MoE alignment for decode B=1..8, MI355X HIP kernel.

Drop-in for `titan_moe_align_small` of kernels/titan_moe_align.py:49-81: the
same contract checks (ValueError), the same three int32 outputs, bit-exact
with the stable baseline (benchmarks/moe_align.py:23-31).  Exact target: 288
experts, top-k 8, block size 8, no expert-parallel map; invalid routes are
ignored.  The kernel (csrc/moe_align.hip) runs one wave64 on the caller's
current stream; `num_warps` is validated as in the reference and does not
change the result (one 64-lane wavefront covers all <= 64 routes).
"""
import torch

import _glm53_lib as _lib


def titan_moe_align_small(
    topk_ids,
    block_size=8,
    num_experts=288,
    expert_map=None,
    pad_sorted_ids=False,
    ignore_invalid_experts=True,
    *,
    num_warps=None,
):
    """Return exactly the stable baseline's three tensors, including padding."""
    if (topk_ids.ndim != 2 or not 1 <= topk_ids.shape[0] <= 8
            or topk_ids.shape[1] != 8 or block_size != 8 or num_experts != 288
            or expert_map is not None or not ignore_invalid_experts):
        raise ValueError('Titan small alignment requires B1..8/top8/E288/block8/EPoff/ignore-invalid')
    if not topk_ids.is_cuda or not topk_ids.is_contiguous():
        raise ValueError('Titan small alignment requires contiguous CUDA route IDs')
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError('Route IDs must be int32 or int64')
    routes = topk_ids.numel()
    # R * 8 entries already cover every padded layout for R < 288, so
    # pad_sorted_ids does not change the result.
    sorted_ids = torch.empty(routes * 8, dtype=torch.int32, device=topk_ids.device)
    expert_ids = torch.empty(routes, dtype=torch.int32, device=topk_ids.device)
    postpad = torch.empty(1, dtype=torch.int32, device=topk_ids.device)
    if num_warps is None:
        num_warps = 1 if routes <= 16 else 4
    if num_warps not in (1, 2, 4):
        raise ValueError('Candidate warp counts are 1, 2, or 4')
    L = _lib.load()
    with torch.cuda.device(topk_ids.device):
        rc = L.glm53_moe_align_small(topk_ids.data_ptr(), int(topk_ids.dtype == torch.int64), routes,
                                     sorted_ids.data_ptr(), expert_ids.data_ptr(), postpad.data_ptr(),
                                     _lib.stream_handle(topk_ids.device))
    _lib.check(rc, "glm53_moe_align_small")
    return sorted_ids, expert_ids, postpad
