"""CPU checks of the drop-in boundary: the C ABI library loads and exports what
include/glm53.h declares, host-side argument errors, and the Python
contract errors of the three reference entry points.  No kernel is launched."""
import ctypes
import re
import sys
import types
from pathlib import Path
from unittest.mock import patch

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "glm53.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(glm53_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import _glm53_lib
    lib = _glm53_lib.load()
    names = declared_functions()
    assert set(names) == set(_glm53_lib.EXPORTED)
    for n in names:
        assert hasattr(lib, n), n
    assert lib.glm53_abi_version() == 3


def test_host_side_argument_errors():
    import _glm53_lib
    L = _glm53_lib.load()
    fake = ctypes.c_void_p(0x10000)   # never dereferenced: every call below fails validation
    assert L.glm53_moe_align_small(None, 0, 8, None, None, None, None) == -1
    assert L.glm53_moe_align_small(fake, 0, 0, fake, fake, fake, None) == -2
    assert L.glm53_moe_align_small(fake, 0, 65, fake, fake, fake, None) == -2
    assert L.glm53_store_int8(fake, 512, fake, 135168, 528, 256, 1024, fake, 1, -1, None) == -2
    assert L.glm53_store_int8(fake, 512, fake, 135168, 528, 0, 1024, fake, 1, 4, None) == -2
    assert L.glm53_store_int8(None, 512, fake, 135168, 528, 256, 1024, fake, 1, 4, None) == -1
    assert L.glm53_store_int8(fake, 512, fake, 135168, 528, 256, 1024, fake, 1, 0, None) == 0
    # misaligned q / row stride
    mis = ctypes.c_void_p(0x10008)
    assert L.glm53_sparse_mla(mis, 8192, 512, fake, 528, 10, fake, 2176, 1, 16, 2176, 0.04, 1,
                              None, 0, fake, 8192, 512, None) == -3
    assert L.glm53_sparse_mla(fake, 8192, 512, fake, 520, 10, fake, 2176, 1, 16, 2176, 0.04, 1,
                              None, 0, fake, 8192, 512, None) == -3
    # split path without workspace
    assert L.glm53_sparse_mla(fake, 8192, 512, fake, 528, 10, fake, 2176, 1, 16, 2176, 0.04, 4,
                              None, 0, fake, 8192, 512, None) == -4
    assert L.glm53_sparse_mla(fake, 8192, 512, fake, 528, 10, fake, 2176, 0, 16, 2176, 0.04, 4,
                              None, 0, fake, 8192, 512, None) == 0
    assert L.glm53_sparse_mla_workspace_bytes(1, 16, 1) == 0
    assert L.glm53_sparse_mla_workspace_bytes(2, 16, 4) == 2 * 4 * 16 * (512 * 4 + 4)
    assert L.glm53_sparse_mla_workspace_bytes(1, 20, 2) == 2 * 32 * (512 * 4 + 4)
    for code in (0, -1, -2, -3, -4, -5):
        assert L.glm53_error_string(code)


def test_moe_contract_errors_on_cpu():
    import torch
    from titan_moe_align import titan_moe_align_small
    ok = torch.zeros(2, 8, dtype=torch.int32)
    bad_cases = [
        (torch.zeros(16, dtype=torch.int32), {}),           # ndim
        (torch.zeros(9, 8, dtype=torch.int32), {}),         # B > 8
        (torch.zeros(0, 8, dtype=torch.int32), {}),         # B < 1
        (torch.zeros(2, 4, dtype=torch.int32), {}),         # top-k
        (ok, {"block_size": 16}),
        (ok, {"num_experts": 256}),
        (ok, {"expert_map": ok}),
        (ok, {"ignore_invalid_experts": False}),
        (ok, {}),                                           # CPU tensor
    ]
    for ids, kw in bad_cases:
        with pytest.raises(ValueError):
            titan_moe_align_small(ids, **kw)


def test_mla_and_writer_contract_assertions_on_cpu():
    import torch
    from titan_kv import store_int8
    from titan_mla import triton_mla_sparse_attention, _choose_num_kv_splits
    kv = torch.zeros(256, 1, 528, dtype=torch.int8)
    q = torch.zeros(1, 16, 512, dtype=torch.bfloat16)
    idx = torch.zeros(1, 1, 2176, dtype=torch.int32)
    with pytest.raises(AssertionError):
        triton_mla_sparse_attention(torch.zeros(1, 16, 256, dtype=torch.bfloat16), kv, idx, 0.04)
    with pytest.raises(AssertionError):
        triton_mla_sparse_attention(q, torch.zeros(256, 1, 512, dtype=torch.int8), idx, 0.04)
    with pytest.raises(AssertionError):
        triton_mla_sparse_attention(q, kv, torch.zeros(1, 1, 100, dtype=torch.int32), 0.04)
    with pytest.raises(NotImplementedError):
        triton_mla_sparse_attention(torch.zeros(1, 16, 576, dtype=torch.bfloat16),
                                    torch.zeros(256, 1, 576, dtype=torch.bfloat16), idx, 0.04)
    with pytest.raises(AssertionError):
        store_int8(torch.zeros(4, 256, dtype=torch.bfloat16), torch.zeros(1, 256, 528, dtype=torch.uint8),
                   torch.arange(4))
    with pytest.raises(AssertionError):
        store_int8(torch.zeros(4, 512, dtype=torch.bfloat16), torch.zeros(1, 256, 528, dtype=torch.uint8),
                   torch.arange(5))
    assert [_choose_num_kv_splits(t, 1, 2176, 70) for t in (1, 6, 8, 2048)] == [32, 8, 8, 1]


def test_library_split_policy_table():
    """The library's auto split count (_choose_num_kv_splits_mi355x): capped
    at tokens x head groups x splits <= CUs and, with more than one (token,
    head group) unit, two 32-key tiles per split; the fewest tiles per split
    under the cap, then the fewest splits giving that many.  Hand table at
    256 CUs (and 70)."""
    from titan_mla import _choose_num_kv_splits_mi355x as pick
    table = {
        (1, 1, 2176, 256): 68,            # one unit: 68 one-tile splits
        (2, 1, 2176, 256): 34, (3, 1, 2176, 256): 34, (4, 1, 2176, 256): 34,
        (1, 2, 2176, 256): 34,            # two head groups: two units
        (8, 1, 2176, 256): 23,            # cap 32 -> 3 tiles per split -> ceil(68 / 3) = 23
        (5, 1, 2176, 256): 23, (6, 1, 2176, 256): 23, (7, 1, 2176, 256): 23,   # sized as 8 tokens
        (7, 2, 2176, 256): 17,            # two head groups: 14 units, cap 18 -> 4 tiles per split -> 17
        (16, 1, 2176, 256): 14,           # cap 16 -> 5 tiles per split -> 14
        (8, 4, 2176, 256): 8,             # 32 units: cap 8 -> 9 tiles per split -> 8
        (256, 1, 2176, 256): 1, (2048, 1, 2176, 256): 1, (300, 1, 2176, 256): 1,
        (1, 1, 32, 256): 1,               # one tile: nothing to split
        (1, 1, 64, 256): 2, (1, 1, 96, 256): 3, (1, 1, 128, 256): 4,
        (2, 1, 64, 256): 1, (2, 1, 128, 256): 2,
        (1, 1, 2150, 256): 1,             # not a multiple of 32
        (1, 1, 16384, 256): 256,          # 512 tiles: 256 splits of 2 (the merge's loop path)
        (1, 1, 2176, 70): 68,             # 68 <= 70
        (3, 1, 2176, 70): 23,             # cap 23 -> 3 tiles per split -> 23
        (0, 1, 2176, 256): 1,
        (1, 1, 0, 256): 1, (8, 1, 0, 256): 1,   # no indices: one (empty) split
    }
    assert {k: pick(*k) for k in table} == table


def test_import_does_not_touch_cuda():
    """Mirrors tests/test_cpu_contracts.py:33-53: importing the entry-point
    modules must not query the device."""
    fake_torch = types.ModuleType("torch")
    fake_torch.Tensor = object

    class NoCUDA:
        def __getattr__(self, name):
            raise AssertionError(f"import-time torch.cuda access: {name}")

    fake_torch.cuda = NoCUDA()
    import importlib.util
    pkg = ROOT / "glm-5.3-kernels_amd"
    with patch.dict(sys.modules, {"torch": fake_torch}):
        for fname, exported in (("titan_kv.py", "store_int8"),
                                ("titan_mla.py", "triton_mla_sparse_attention"),
                                ("titan_moe_align.py", "titan_moe_align_small"),
                                ("sparse_utils.py", "triton_convert_req_index_to_global_index"),
                                ("titan_moe_w4a16.py", "fused_moe_w4a16"),
                                ("sparse_indexer.py", "fp8_paged_mqa_logits")):
            spec = importlib.util.spec_from_file_location("isolated_" + fname[:-3], pkg / fname)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            assert callable(getattr(mod, exported))


def test_product_does_not_import_oracle():
    for f in (ROOT / "glm-5.3-kernels_amd").rglob("*.py"):
        text = f.read_text()
        assert "import oracle" not in text and "from oracle" not in text, f


def test_paged_entry_points_host_errors():
    import _glm53_lib
    L = _glm53_lib.load()
    fake = ctypes.c_void_p(0x10000)
    # convert: null req_id, zero block size, page rows below block size, T = 0
    assert L.glm53_convert_req_index(None, fake, 2, 8, 8, fake, 64, fake, 64, 1, 64, 16, 16, None) == -1
    assert L.glm53_convert_req_index(fake, fake, 2, 8, 8, fake, 64, fake, 64, 1, 64, 0, 16, None) == -2
    assert L.glm53_convert_req_index(fake, fake, 2, 8, 8, fake, 64, fake, 64, 1, 64, 16, 15, None) == -2
    assert L.glm53_convert_req_index(fake, fake, 2, 8, 8, fake, 64, fake, 64, 0, 64, 16, 16, None) == 0
    # paged attention: argument errors before any launch
    args = [fake, 8192, 512, fake, 36864, 528, 64, fake, 2176, fake, fake, 2, 8, 8, 64,
            1, 16, 2176, 0.04, 4, None, 0, fake, 8192, 512, None]
    assert L.glm53_sparse_mla_paged(*args) == -4                        # no workspace
    bad = list(args); bad[9] = None
    assert L.glm53_sparse_mla_paged(*bad) == -1                         # null req_id
    bad = list(args); bad[14] = 0
    assert L.glm53_sparse_mla_paged(*bad) == -2                         # block size 0
    bad = list(args); bad[4] = 36864 + 8
    assert L.glm53_sparse_mla_paged(*bad) == -3                         # page stride not 16-byte aligned
    bad = list(args); bad[4] = 63 * 528
    assert L.glm53_sparse_mla_paged(*bad) == -2                         # 64 rows do not fit the page
    bad = list(args); bad[15] = 0
    assert L.glm53_sparse_mla_paged(*bad) == 0                          # T = 0


def test_flat_kv_row_view_on_cpu():
    import torch
    from sparse_utils import flat_kv_row_view
    raw = torch.arange(5 * 7 * 3, dtype=torch.int32).reshape(5, 7, 3)
    paged = raw[:, :4, :]                     # 4 tokens per block, pages of 7 rows
    rows, stride = flat_kv_row_view(paged, 4)
    assert stride == 7 and rows.shape == (4 * 7 + 4, 3)
    for b in range(5):
        for i in range(4):
            assert torch.equal(rows[b * 7 + i], paged[b, i])
    with pytest.raises(ValueError):
        flat_kv_row_view(paged, 8)
    with pytest.raises(ValueError):
        flat_kv_row_view(torch.zeros(4, 4, 3)[:, :, :2], 4)   # rows not contiguous


def test_convert_contract_on_cpu():
    import torch
    from sparse_utils import triton_convert_req_index_to_global_index as conv
    req = torch.zeros(2, dtype=torch.int32)
    bt = torch.zeros(1, 4, dtype=torch.int32)
    idx = torch.zeros(2, 256, dtype=torch.int32)
    with pytest.raises(AssertionError):
        conv(req, bt, idx, BLOCK_SIZE=64, NUM_TOPK_TOKENS=128)
    with pytest.raises(AssertionError):
        conv(req.long(), bt, idx, BLOCK_SIZE=64, NUM_TOPK_TOKENS=256)
    with pytest.raises(NotImplementedError):
        conv(req, bt, idx, BLOCK_SIZE=64, NUM_TOPK_TOKENS=256, HAS_PREFILL_WORKSPACE=True)


def test_moe_w4a16_host_errors():
    """Argument errors of the W4A16 MoE entry points are caught on the host
    before any launch (no device needed)."""
    import _glm53_lib
    L = _glm53_lib.load()
    fake = ctypes.c_void_p(0x10000)
    mis = ctypes.c_void_p(0x10008)
    # repack: null, shapes, alignment
    assert L.glm53_moe_w4a16_repack(None, fake, 288, 1024, 4096, fake, fake, None) == -1
    assert L.glm53_moe_w4a16_repack(fake, None, 288, 1024, 4096, fake, fake, None) == -1
    assert L.glm53_moe_w4a16_repack(fake, fake, 288, 1000, 4096, fake, fake, None) == -2
    assert L.glm53_moe_w4a16_repack(fake, fake, 288, 1024, 4000, fake, fake, None) == -2
    assert L.glm53_moe_w4a16_repack(fake, fake, 0, 1024, 4096, fake, fake, None) == -2
    assert L.glm53_moe_w4a16_repack(fake, fake, 288, 1024, 4096, mis, fake, None) == -3
    # gate/up: x, sx, w13, s13, sorted, experts, R, topk, E, N, K, clamp, act, stream
    args = [fake, 4096, fake, fake, fake, fake, 64, 8, 288, 512, 4096, 10.0, fake, None]
    bad = lambda i, v: L.glm53_moe_w4a16_gate_up(*(args[:i] + [v] + args[i + 1:]))
    assert bad(0, None) == -1
    assert bad(9, 500) == -2            # N not a multiple of 16
    assert bad(10, 4000) == -2          # K not a multiple of 128
    assert bad(1, 4000) == -2           # row stride below K
    assert bad(11, 0.0) == -2           # clamp limit must be > 0
    assert bad(11, float("nan")) == -2
    assert bad(0, mis) == -3
    assert bad(1, 4100) == -3           # row stride breaks 16-byte rows
    # down: act, w2, s2, ids, i64, sid_t, w, sw_t, T, topk, E, N, K, out, so, stream
    args = [fake, fake, fake, fake, 0, 8, fake, 8, 8, 8, 288, 512, 4096, fake, 4096, None]
    bad = lambda i, v: L.glm53_moe_w4a16_down(*(args[:i] + [v] + args[i + 1:]))
    assert bad(6, None) == -1
    assert bad(9, 9) == -2              # more than 8 routes per token
    assert bad(11, 500) == -2           # N not a multiple of 128
    assert bad(5, 4) == -2              # ids row stride below topk
    assert bad(0, mis) == -3
    # fused: the aligner's contract (1..8 tokens, top-8, 288 experts) and the workspace
    ws = L.glm53_fused_moe_w4a16_workspace_bytes(8, 8, 512)
    assert ws >= 64 * 512 * 2                # the c2 activations of 64 routes
    args = [fake, 4096, fake, fake, fake, fake, fake, 0, fake, 8, 8, 288, 512, 4096, 10.0, fake, ws, fake,
            4096, None]
    bad = lambda i, v: L.glm53_fused_moe_w4a16(*(args[:i] + [v] + args[i + 1:]))
    assert bad(9, 9) == -2              # 9 tokens
    assert bad(10, 4) == -2             # top-4
    assert bad(11, 256) == -2           # 256 experts
    assert bad(16, ws - 1) == -4
    assert bad(15, None) == -1


def test_moe_w4a16_contract_errors_on_cpu():
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16, repack_w4a16
    x = torch.zeros(2, 4096, dtype=torch.bfloat16)
    w13 = torch.zeros(288, 64, 32, 64, 4, dtype=torch.int32)
    w2 = torch.zeros(288, 256, 4, 64, 4, dtype=torch.int32)
    s13 = torch.zeros(288, 64, 32, 16, 4, dtype=torch.bfloat16)
    s2 = torch.zeros(288, 256, 4, 16, 4, dtype=torch.bfloat16)
    tw = torch.zeros(2, 8)
    ids = torch.zeros(2, 8, dtype=torch.int32)
    call = lambda **kw: fused_moe_w4a16(**{**dict(hidden_states=x, w13=w13, w2=w2, w13_scale=s13,
                                                  w2_scale=s2, topk_weights=tw, topk_ids=ids), **kw})
    with pytest.raises(ValueError, match="expert_map"):
        call(expert_map=torch.arange(288))
    with pytest.raises(ValueError, match="router weight"):
        call(apply_router_weight_on_input=True)
    with pytest.raises(ValueError, match="tokens"):
        call(hidden_states=torch.zeros(9, 4096, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="topk_ids"):
        call(topk_ids=torch.zeros(2, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="topk_weights"):
        call(topk_weights=torch.zeros(2, 8, dtype=torch.float16))
    with pytest.raises(ValueError, match="experts"):
        call(w13=w13[:256], w2=w2[:256])
    with pytest.raises(ValueError, match="w13_scale"):
        call(w13_scale=torch.zeros(288, 1024, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="w2"):
        call(w2=torch.zeros(288, 256, 4, 64, 2, dtype=torch.int32))
    with pytest.raises(ValueError, match="clamp_limit"):
        call(clamp_limit=0.0)
    with pytest.raises(ValueError):
        repack_w4a16(torch.zeros(288, 1000, 512, dtype=torch.int32), torch.zeros(288, 1000, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        repack_w4a16(torch.zeros(288, 1024, 512, dtype=torch.int32), torch.zeros(288, 1024, 64, dtype=torch.bfloat16))


def test_indexer_host_errors():
    import _glm53_lib
    L = _glm53_lib.load()
    fake = ctypes.c_void_p(0x10000)
    mis = ctypes.c_void_p(0x10008)
    # q, sq_t, sq_h, kv, page_bytes, bs, nb, w, sw_t, ctx, bt, bt_stride, max_blocks, T, H, D, max_len, clean, out, sl, stream
    args = [fake, 4096, 128, fake, 64 * 132, 64, 100, fake, 32, fake, fake, 16, 16, 8, 32, 128, 1024, 1, fake, 1024, None]
    bad = lambda i, v: L.glm53_fp8_paged_mqa_logits(*(args[:i] + [v] + args[i + 1:]))
    assert bad(0, None) == -1
    assert bad(15, 64) == -2        # head_dim must be 128
    assert bad(14, 24) == -2        # heads a multiple of 16
    assert bad(14, 80) == -2        # at most 64 heads
    assert bad(4, 64 * 132 - 16) == -2   # page smaller than block_size x 132
    assert bad(19, 1000) == -2      # logits row stride below max_len
    assert bad(16, (1 << 30) + 1) == -2   # positions past 2^30
    assert bad(6, 1 << 31) == -2    # block ids past int32
    assert bad(0, mis) == -3
    assert bad(4, 64 * 132 + 8) == -3    # page stride not a multiple of 16
    assert bad(13, 0) == 0          # nothing to do
    # logits, sl, lengths, rows, max_len, k, ws, ws_bytes, out, so, stream
    args = [fake, 1024, fake, 8, 1024, 512, None, 0, fake, 512, None]
    bad = lambda i, v: L.glm53_indexer_topk(*(args[:i] + [v] + args[i + 1:]))
    assert bad(0, None) == -1
    assert bad(5, 0) == -2
    assert bad(5, 2048) == -2       # k above the row length
    assert bad(9, 100) == -2        # output row stride below k
    assert bad(0, ctypes.c_void_p(0x10002)) == -3   # logits not float-aligned
    assert bad(3, 0) == 0
    # long rows run in two stages and need the candidates' workspace
    ws = L.glm53_indexer_topk_workspace_bytes
    assert ws(8, 4096, 512) == 0
    assert ws(8, 65536, 512) == 8 * 8 * 512 * 8           # 8 chunks of 8192, key + position per candidate
    assert ws(8, 16384, 512) == 8 * 4 * 512 * 8           # 4 chunks of 4096
    assert ws(8, 65536, 2048) == 8 * 8 * 2048 * 8         # 8 chunks of 8192
    assert ws(2, 140000, 4096) == 0                       # too many candidates: single-workgroup sweeps
    assert ws(8, 65536, 0) == 0 and ws(-1, 65536, 512) == 0
    big = [fake, 65536, fake, 8, 65536, 512, None, 0, fake, 512, None]
    assert L.glm53_indexer_topk(*big) == -4
    big[6], big[7] = fake, ws(8, 65536, 512) - 1
    assert L.glm53_indexer_topk(*big) == -4


def test_indexer_contract_errors_on_cpu():
    import torch
    from sparse_indexer import fp8_paged_mqa_logits, indexer_topk
    q = torch.zeros(2, 1, 32, 128, dtype=torch.float8_e4m3fn)
    kv = torch.zeros(10, 64, 1, 132, dtype=torch.uint8)
    w = torch.zeros(2, 32)
    ctx = torch.zeros(2, dtype=torch.int32)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="q must be"):
        fp8_paged_mqa_logits(q.float(), kv, w, ctx, bt, 256)
    with pytest.raises(ValueError, match="kv_cache"):
        fp8_paged_mqa_logits(q, kv[..., :128], w, ctx, bt, 256)
    with pytest.raises(ValueError, match="weights"):
        fp8_paged_mqa_logits(q, kv, w[:, :16], ctx, bt, 256)
    with pytest.raises(ValueError, match="context_lens"):
        fp8_paged_mqa_logits(q, kv, w, ctx.long(), bt, 256)
    with pytest.raises(ValueError, match="k <="):
        indexer_topk(torch.zeros(2, 100), ctx, 512)
    with pytest.raises(ValueError, match="lengths"):
        indexer_topk(torch.zeros(2, 1000), ctx.long(), 512)


def test_topk_plans_keep_their_invariants():
    """The two-stage top-k's plan (through the workspace size it needs): when
    it chunks, chunks of 4096, 8192 or 16384 positions, longer than k, at least
    two of them, and at most 32768 candidates for the final workgroup; rows of
    at most 4096 columns never chunk."""
    import _glm53_lib
    L = _glm53_lib.load()
    ws = L.glm53_indexer_topk_workspace_bytes
    for max_len in (1, 100, 4096, 4097, 8191, 20000, 32768, 65536, 65537, 140000, 262144, 1 << 20):
        for k in (1, 7, 512, 2048, 4095, 4096, 8192, 16384, 32768):
            if k > max_len:
                assert ws(3, max_len, k) == 0
                continue
            b = ws(3, max_len, k)
            if max_len <= 4096:
                assert b == 0, (max_len, k)
                continue
            if b == 0:
                continue   # one workgroup over the row, or the sweeping kernel
            per_row = b / 3 / 8 / k          # candidates slots = chunks (rounded workspace aside)
            ok = False
            for p in (8, 16, 32):
                chunk = 512 * p
                chunks = -(-max_len // chunk)
                if chunk > k and chunks >= 2 and chunks * k <= 32768 and ws(3, max_len, k) == -(-(3 * chunks * k * 8) // 256) * 256:
                    ok = True
            assert ok, (max_len, k, per_row)


def test_topk_workspace_query_covers_fewer_rows():
    """glm53_indexer_topk_workspace_bytes(n, ...) is enough for every call of
    at most n rows: the plan moves to 512-thread chunks at 32 rows, whose
    candidates take less room than the latency plan's at 31 rows, so the
    query never shrinks as n grows."""
    import _glm53_lib
    L = _glm53_lib.load()
    ws = L.glm53_indexer_topk_workspace_bytes
    assert ws(31, 16384, 512) == 507904
    assert ws(32, 16384, 512) >= 507904
    for max_len, k in ((16384, 512), (65536, 512), (262144, 512), (65536, 2048), (20000, 100)):
        sizes = [ws(n, max_len, k) for n in range(1, 80)]
        assert all(b >= a for a, b in zip(sizes, sizes[1:])), (max_len, k)


def test_attention_token_limit():
    """Query tokens are the split kernel's grid y: every attention entry
    point rejects more than 65535 with GLM53_ERR_BAD_SHAPE before anything is
    launched (the Python wrappers cut larger calls into ranges)."""
    import _glm53_lib
    L = _glm53_lib.load()
    fake = ctypes.c_void_p(0x10000)
    T = 65536
    assert L.glm53_sparse_mla(fake, 8192, 512, fake, 528, 10, fake, 2176, T, 16, 2176, 0.04, 4,
                              fake, 1 << 40, fake, 8192, 512, None) == -2
    assert L.glm53_sparse_mla_noalloc(fake, 8192, 512, fake, 528, 10, fake, 2176, T, 16, 2176, 0.04, 1,
                                      fake, 8192, 512, None) == -2
    assert L.glm53_sparse_mla_partials(fake, 8192, 512, fake, 528, 10, fake, 2176, T, 16, 2176, 0.04, 4,
                                       fake, 1 << 40, None) == -2
    assert L.glm53_sparse_mla_gather_floor(fake, 8192, 512, fake, 528, 10, fake, 2176, T, 16, 2176, 4,
                                           fake, 1 << 40, None) == -2
    assert L.glm53_sparse_mla_paged(fake, 8192, 512, fake, 33792, 528, 10, fake, 2176, fake, fake, 1, 4, 4, 64,
                                    T, 16, 2176, 0.04, 4, fake, 1 << 40, fake, 8192, 512, None) == -2
    assert L.glm53_sparse_mla_pooled(fake, 8192, 512, fake, 33792, 528, 10, fake, 512, 512, None, 4,
                                     fake, fake, 1, 4, 4, 64, T, 16, 2176, 0.04, 4, fake, 1 << 40,
                                     fake, 8192, 512, None) == -2


def test_stream_probe_argument_checks():
    """The streaming probe validates before anything is launched: unknown
    kind, null pointers, sizes that are not a positive multiple of 16 and
    pointers off 16-byte alignment."""
    import _glm53_lib
    L = _glm53_lib.load()
    a, b = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x20000)
    assert L.glm53_stream_probe(3, a, b, 1 << 20, None) == -2
    assert L.glm53_stream_probe(-1, a, b, 1 << 20, None) == -2
    assert L.glm53_stream_probe(0, None, b, 1 << 20, None) == -1
    assert L.glm53_stream_probe(2, a, None, 1 << 20, None) == -1
    assert L.glm53_stream_probe(1, a, b, 8, None) == -2
    assert L.glm53_stream_probe(1, a, b, (1 << 20) + 4, None) == -2
    assert L.glm53_stream_probe(0, ctypes.c_void_p(0x10008), b, 1 << 20, None) == -3
    assert L.glm53_stream_probe(2, a, ctypes.c_void_p(0x20004), 1 << 20, None) == -3
