"""CPU checks of the C ABI (``include/sqa.h`` / ``libsqa.so``): no kernel launches.

The library must load, export every function the header declares, and reject
bad arguments with the documented status codes before touching the GPU.
"""

import ctypes
import re
from pathlib import Path

import pytest

from small_q_attention_amd import _lib, build

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sqa.h"

SQA_OK, SQA_ERR_INVALID, SQA_ERR_UNSUPPORTED, SQA_ERR_WORKSPACE = 0, 1, 2, 3


def declared_functions():
    text = HEADER.read_text()
    body = text[text.index('extern "C" {'):]
    return sorted(set(re.findall(r"\b(sqa_[a-z0-9_]+)\s*\(", body)))


@pytest.fixture(scope="module")
def lib():
    if build.is_stale():
        build.build()
    return _lib.load()


def test_header_declares_the_bound_functions():
    assert declared_functions() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(_lib.library_path()))
    for name in declared_functions():
        assert hasattr(raw, name), name


def test_version_and_empty_error(lib):
    assert lib.sqa_version().decode().startswith("sqa ")
    assert isinstance(lib.sqa_last_error(), bytes)


def test_workspace_bytes(lib):
    # Fixed plan: rows = q_len * group; items = B * Hkv * splits * rows; 130 floats each.
    assert lib.sqa_workspace_bytes(16, 8, 32, 8, 128, 1, 2048) == 0
    assert lib.sqa_workspace_bytes(16, 8, 32, 8, 128, 16, 128) == 16 * 8 * 16 * 32 * 130 * 4
    assert lib.sqa_workspace_bytes(1, 2, 32, 8, 128, 3, 4) == 1 * 8 * 3 * 8 * 130 * 4
    assert lib.sqa_workspace_bytes(0, 2, 32, 8, 128, 3, 4) == 0
    # Balanced plan (pages_per_split 0): num_splits slots shared by the batch,
    # plus one (first slot, count) pair of int32 per sequence, the paired items'
    # 16-byte delta record and two 8-byte loop-time records per slot.
    assert lib.sqa_workspace_bytes(16, 8, 32, 8, 128, 272, 0) == \
        272 * 8 * 32 * 130 * 4 + 16 * 8 + 16 + 272 * 16
    assert lib.sqa_workspace_bytes(2, 2, 32, 8, 128, 1, 0) == \
        1 * 8 * 8 * 130 * 4 + 2 * 8 + 16 + 16
    # -P: the balanced plan expecting P pages per sequence; the same workspace.
    assert lib.sqa_workspace_bytes(2, 2, 32, 8, 128, 3, -7) == \
        lib.sqa_workspace_bytes(2, 2, 32, 8, 128, 3, 0) == 3 * 8 * 8 * 130 * 4 + 2 * 8 + 16 + 48
    # Other head dims: head_dim + 2 floats per item.
    assert lib.sqa_workspace_bytes(1, 2, 32, 8, 64, 3, 4) == 1 * 8 * 3 * 8 * 66 * 4
    assert lib.sqa_workspace_bytes(1, 2, 32, 8, 256, 3, 4) == 1 * 8 * 3 * 8 * 258 * 4
    assert lib.sqa_workspace_bytes(1, 2, 32, 8, 0, 3, 4) == 0


def _plan(lib, **kw):
    args = dict(device=0, batch=4, q_len=4, hq=32, hkv=8, hd=128, max_seq_len=8192,
                max_pages=512, chunk_keys=512)
    args.update(kw)
    ns, pps = ctypes.c_int(-7), ctypes.c_int(-7)
    rc = lib.sqa_plan_splits(args["device"], args["batch"], args["q_len"], args["hq"], args["hkv"],
                             args["hd"], args["max_seq_len"], args["max_pages"],
                             args["chunk_keys"], ctypes.byref(ns), ctypes.byref(pps))
    return rc, ns.value, pps.value


def test_plan_with_explicit_chunk_keys(lib):
    # Reference meaning (csrc/small_q_attention_ext.cu:1177): ceil(longest / chunk) chunks.
    assert _plan(lib) == (SQA_OK, 16, 32)
    assert _plan(lib, chunk_keys=128, max_seq_len=33, max_pages=3) == (SQA_OK, 1, 3)
    assert _plan(lib, chunk_keys=1 << 20, max_seq_len=8192) == (SQA_OK, 1, 512)
    assert _plan(lib, chunk_keys=100, max_seq_len=1000, max_pages=63) == (SQA_OK, 9, 7)
    # Unknown max_seq_len: the plan covers the whole block-table row.
    assert _plan(lib, chunk_keys=512, max_seq_len=0, max_pages=100) == (SQA_OK, 4, 32)
    # A split owns at most 2048 pages (the kernel's LDS page-id table).
    assert _plan(lib, chunk_keys=1 << 20, max_seq_len=65536, max_pages=4096) == (SQA_OK, 2, 2048)


def test_plan_rejects_bad_arguments(lib):
    assert _plan(lib, batch=0)[0] == SQA_ERR_INVALID
    assert _plan(lib, chunk_keys=-1)[0] == SQA_ERR_INVALID
    assert _plan(lib, max_pages=0)[0] == SQA_ERR_INVALID
    rc = lib.sqa_plan_splits(0, 1, 2, 32, 8, 128, 16, 1, 16, None, None)
    assert rc == SQA_ERR_INVALID


def _call(lib, **kw):
    # Fake, 16-byte aligned device addresses: validation fails before any is used.
    args = dict(q=16, k=16, v=16, bt=16, sl=16, out=16, ws=None, ws_bytes=0, batch=1, q_len=2,
                hq=32, hkv=8, dim=128, num_pages=4, page=16, max_pages=2, splits=1, pps=2)
    args.update(kw)
    return lib.sqa_paged_mtp_attention(
        args["q"], args["k"], args["v"], args["bt"], args["sl"], args["out"], args["ws"],
        args["ws_bytes"], args["batch"], args["q_len"], args["hq"], args["hkv"], args["dim"],
        args["num_pages"], args["page"], args["max_pages"], args["splits"], args["pps"], None, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(q=None), SQA_ERR_INVALID, "null"),
    (dict(batch=0), SQA_ERR_INVALID, "positive"),
    (dict(num_pages=0), SQA_ERR_INVALID, "empty"),
    (dict(hkv=5), SQA_ERR_INVALID, "divisible"),
    (dict(dim=96), SQA_ERR_UNSUPPORTED, "head_dim"),
    (dict(dim=512), SQA_ERR_UNSUPPORTED, "head_dim"),
    # head_dim 256 holds at most 32 rows per kv head.
    (dict(dim=256, q_len=16), SQA_ERR_UNSUPPORTED, "exceeds 32 at head_dim 256"),
    (dict(page=24), SQA_ERR_UNSUPPORTED, "page_size"),
    (dict(page=512), SQA_ERR_UNSUPPORTED, "page_size"),
    # 64-token pages: the balanced plan's slot bound counts 16-token pages.
    (dict(pps=0, batch=4, splits=7, max_pages=513, page=64, ws=16, ws_bytes=1 << 40),
     SQA_ERR_INVALID, "num_splits >= batch + 5"),
    (dict(q_len=32), SQA_ERR_UNSUPPORTED, "exceeds"),
    (dict(splits=0), SQA_ERR_INVALID, "positive"),
    (dict(pps=2049), SQA_ERR_INVALID, "exceeds"),
    # -P: balanced plan expecting P pages per sequence; P beyond the block-table row
    # (max_pages 2 x 16-token pages) is refused.
    (dict(pps=-3, batch=2, splits=3, ws=16, ws_bytes=1 << 40), SQA_ERR_INVALID, "expects 3 pages"),
    (dict(pps=-1, batch=1, splits=1, ws=16, ws_bytes=1 << 40), SQA_ERR_INVALID, "num_splits >="),
    # Balanced plan: at most 256 sequences, at least one spare slot per sequence
    # plus enough slots to keep every split within 2048 pages.
    (dict(pps=0, batch=257, splits=600, ws=16, ws_bytes=1 << 40), SQA_ERR_INVALID, "batch <= 256"),
    (dict(pps=0, batch=4, splits=4, ws=16, ws_bytes=1 << 40), SQA_ERR_INVALID, "num_splits >="),
    (dict(pps=0, batch=4, splits=7, max_pages=2049, ws=16, ws_bytes=1 << 40), SQA_ERR_INVALID,
     "num_splits >= batch + 5"),
    (dict(pps=0, batch=2, splits=3, ws=None), SQA_ERR_WORKSPACE, "workspace"),
    (dict(splits=2, ws=None), SQA_ERR_WORKSPACE, "workspace"),
    (dict(splits=2, ws=16, ws_bytes=100), SQA_ERR_WORKSPACE, "workspace"),
    (dict(splits=2, ws=24, ws_bytes=1 << 40), SQA_ERR_WORKSPACE, "16-byte aligned"),
    (dict(k=24), SQA_ERR_INVALID, "16-byte aligned"),
    (dict(q=24), SQA_ERR_INVALID, "query must be 16-byte"),
    (dict(out=20), SQA_ERR_INVALID, "output 8-byte aligned"),
    (dict(bt=18), SQA_ERR_INVALID, "4-byte aligned"),
    (dict(sl=17), SQA_ERR_INVALID, "4-byte aligned"),
    # Partial sums travel through 32-bit buffer offsets: a plan whose partials
    # pass 4 GiB (16 x 2048 one-page splits x 8 kv heads x 64 rows x 256 bytes)
    # is refused before anything is launched.
    (dict(batch=16, q_len=16, max_pages=2048, splits=2048, pps=1, ws=16, ws_bytes=1 << 40),
     SQA_ERR_INVALID, "partials"),
])
def test_launch_rejects_bad_arguments_without_a_gpu(lib, kw, code, msg):
    # Validation runs before any HIP call, so these pointers are never touched.
    assert _call(lib, **kw) == code
    assert msg in lib.sqa_last_error().decode()


def _general(lib, **kw):
    """sqa_paged_attention with fake aligned pointers and the given overrides."""
    a = _lib.AttentionArgs()
    a.struct_size = ctypes.sizeof(_lib.AttentionArgs)
    a.query = a.output = a.block_tables = a.seq_lens = 16
    a.kv = _lib.KVCache(16, 16, 4, 16 * 8 * 128, 8 * 128, 128)
    a.max_pages, a.scale, a.out_scale = 2, 128 ** -0.5, 1.0
    a.batch, a.q_len, a.num_query_heads, a.num_kv_heads = 1, 2, 32, 8
    a.head_dim, a.page_size, a.num_splits, a.pages_per_split = 128, 16, 1, 2
    for k, v in kw.items():
        if k.startswith("kv_"):
            setattr(a.kv, k[3:], v)
        else:
            setattr(a, k, v)
    return lib.sqa_paged_attention(ctypes.byref(a))


@pytest.mark.parametrize("kw,code,msg", [
    (dict(struct_size=8), SQA_ERR_INVALID, "struct_size"),
    (dict(kv_k=None), SQA_ERR_INVALID, "null"),
    (dict(kv_token_stride=100), SQA_ERR_INVALID, "multiples of 8"),
    (dict(kv_head_stride=-8), SQA_ERR_INVALID, "multiples of 8"),
    (dict(kv_v=40), SQA_ERR_INVALID, "16-byte aligned"),
    (dict(kv_token_stride=1 << 27), SQA_ERR_INVALID, "2 GiB"),
    (dict(draft_mask=16, mask_words=0), SQA_ERR_INVALID, "draft_mask"),
    (dict(draft_mask=16, mask_words=3), SQA_ERR_INVALID, "draft_mask"),
    (dict(scale=0.0), SQA_ERR_INVALID, "scale"),
    (dict(out_scale=float("inf")), SQA_ERR_INVALID, "out_scale"),
    (dict(head_dim=32), SQA_ERR_UNSUPPORTED, "head_dim"),
    (dict(num_splits=2), SQA_ERR_WORKSPACE, "workspace"),
])
def test_general_entry_rejects_bad_arguments_without_a_gpu(lib, kw, code, msg):
    assert _general(lib, **kw) == code
    assert msg in lib.sqa_last_error().decode()


def test_general_entry_struct_matches_the_header(lib):
    # A struct of the wrong size is refused; the right one, and the layout that
    # stops before `flags` (read as flags = 0), get past that check (and are then
    # refused for a missing workspace, before any device access).
    size = ctypes.sizeof(_lib.AttentionArgs)
    legacy = _lib.AttentionArgs.flags.offset
    assert legacy == size - 8
    for bad in (size - 4, size + 8, legacy - 8):
        assert _general(lib, struct_size=bad) == SQA_ERR_INVALID
        assert "struct_size" in lib.sqa_last_error().decode()
    assert _general(lib, num_splits=2) == SQA_ERR_WORKSPACE
    assert _general(lib, struct_size=legacy, num_splits=2) == SQA_ERR_WORKSPACE
    # The legacy layout never reads `flags`: a junk value there is not seen.
    assert _general(lib, struct_size=legacy, num_splits=2, flags=0x7f) == SQA_ERR_WORKSPACE


def test_general_entry_flags(lib):
    header = HEADER.read_text()
    assert "#define SQA_FLAG_ADAPTIVE_PAIRS 1" in header
    assert _lib.FLAG_ADAPTIVE_PAIRS == 1
    assert _general(lib, flags=2) == SQA_ERR_INVALID
    assert "flags" in lib.sqa_last_error().decode()
    assert _general(lib, flags=_lib.FLAG_ADAPTIVE_PAIRS, num_splits=2) == SQA_ERR_WORKSPACE


def test_noalloc_rejects_plans_beyond_its_scratch_before_any_device_call(lib):
    """SQA_NOALLOC_SCRATCH_BYTES (64 MiB) bounds the plan; larger plans fail with
    SQA_ERR_WORKSPACE before the library touches a device (so this runs without a GPU)."""
    need = lib.sqa_workspace_bytes(1, 16, 32, 8, 128, 2048, 1)
    assert need > (64 << 20)
    rc = lib.sqa_paged_mtp_attention_noalloc(None, None, None, None, None, None, 1, 16, 32, 8,
                                             128, 4096, 16, 2048, 2048, 1, None)
    assert rc == SQA_ERR_WORKSPACE
    assert b"no-allocation" in lib.sqa_last_error()
    header = HEADER.read_text()
    assert "#define SQA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)" in header


@pytest.mark.parametrize("dtype", ["float8_e4m3fn", "bfloat16", "float32"])
def test_fp16_launcher_refuses_other_element_types(dtype):
    """``sqa_paged_mtp_attention`` reads fp16 through bare pointers: the Python
    launcher refuses any other cache type before the call (an e4m3 pool read as
    fp16 would be read past its end)."""
    import torch

    q = torch.zeros(1, 2, 32, 128, dtype=torch.float16)
    k = torch.zeros(4, 16, 8, 128, dtype=getattr(torch, dtype))
    bt = torch.zeros(1, 4, dtype=torch.int32)
    sl = torch.full((1,), 64, dtype=torch.int32)
    with pytest.raises(TypeError, match="launch_general"):
        _lib.launch(q, k, k, bt, sl, torch.empty_like(q), None, 1, 4, 0)
