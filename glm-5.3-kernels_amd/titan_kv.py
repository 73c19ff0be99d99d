# SPDX-License-Identifier: Apache-2.0
"""Per-token symmetric INT8 latent KV writer, MI355X (gfx950) HIP kernel.

Drop-in for `store_int8` of kernels/titan_kv.py:23-28: same name, arguments
and assertions.  The arithmetic runs in the HIP kernel glm53_store_int8
(csrc/store_int8.hip) on the caller's current stream; there is no host sync,
so the call is graph-capturable.

Row format (528 bytes): 512 int8 codes q = clamp(rint(x / s), -127, 127),
fp32 s = max(max|x| / 127, 1e-12) at byte 512, 12 zero bytes.  The quotient
x / s is the correctly rounded IEEE fp32 one.  A negative slot is skipped.

Differences from the reference, all on inputs it leaves undefined:
* a slot at or beyond the cache's capacity (num_blocks * block_size) is
  skipped instead of writing outside the cache;
* the cache may have any 1-byte dtype (it is viewed as int8, as the
  reference does) and its strides are taken in bytes from that view.
"""
import torch

import _glm53_lib as _lib

_LATENT = 512
_ROW_BYTES = 528


def store_int8(x, cache, slots):
    assert x.shape[-1] == _LATENT and cache.shape[-1] == _ROW_BYTES
    slots = slots.flatten()
    assert slots.numel() <= x.shape[0]
    n = slots.numel()
    if n == 0:
        return
    if not (x.is_cuda and cache.is_cuda and slots.is_cuda):
        raise ValueError("store_int8 requires CUDA (HIP) tensors")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"store_int8 expects bf16 latents, got {x.dtype}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    if slots.dtype not in (torch.int32, torch.int64):
        slots = slots.to(torch.int64)
    slots = slots.contiguous()
    c8 = cache.view(torch.int8)
    block = cache.shape[1]
    capacity = cache.shape[0] * block
    L = _lib.load()
    with torch.cuda.device(x.device):
        rc = L.glm53_store_int8(x.data_ptr(), x.stride(0), c8.data_ptr(), c8.stride(0), c8.stride(1),
                                block, capacity, slots.data_ptr(), int(slots.dtype == torch.int64), n,
                                _lib.stream_handle(x.device))
    _lib.check(rc, "glm53_store_int8")
