"""The torch custom ops the traced (torch.compile / torch.export) path calls, checked
without a GPU: registered under the ``sqa`` namespace with the argument lists the
callers pass, and their fake implementations shaping the output on meta tensors
(which is all a tracer asks of them)."""

import pytest

torch = pytest.importorskip("torch")

from small_q_attention_amd import _op  # noqa: E402,F401  (registers the ops)


def _meta_inputs(batch=3, q_len=8, hq=32, hkv=8, d=128, pages=40, width=12, dtype=None):
    dtype = dtype or torch.float16
    q = torch.empty(batch, q_len, hq, d, dtype=dtype, device="meta")
    k = torch.empty(pages, 16, hkv, d, dtype=dtype, device="meta")
    v = torch.empty(pages, 16, hkv, d, dtype=dtype, device="meta")
    bt = torch.empty(batch, width, dtype=torch.int32, device="meta")
    sl = torch.empty(batch, dtype=torch.int32, device="meta")
    return q, k, v, bt, sl


@pytest.mark.parametrize("name,args", [
    ("paged_mtp_attention", ("query", "key_cache", "value_cache", "block_tables", "seq_lens",
                             "num_splits", "pages_per_split")),
    ("paged_mtp_attention_planned", ("query", "key_cache", "value_cache", "block_tables",
                                     "seq_lens", "max_seq_len", "chunk_keys")),
    ("paged_attention_planned", ("query", "k_view", "v_view", "block_tables", "seq_lens",
                                 "draft_mask", "scale", "out_scale", "max_seq_len")),
])
def test_ops_are_registered_with_their_arguments(name, args):
    op = getattr(torch.ops.sqa, name).default
    assert tuple(a.name for a in op._schema.arguments) == args
    assert len(op._schema.returns) == 1
    assert not any(a.alias_info is not None and a.alias_info.is_write
                   for a in op._schema.arguments), "no op writes its inputs"


def test_fake_implementations_shape_the_output():
    q, k, v, bt, sl = _meta_inputs()
    out = torch.ops.sqa.paged_mtp_attention(q, k, v, bt, sl, 144, -512)
    assert out.shape == q.shape and out.dtype == q.dtype and out.device.type == "meta"
    out = torch.ops.sqa.paged_mtp_attention_planned(q, k, v, bt, sl, 3000, 0)
    assert out.shape == q.shape and out.dtype == q.dtype
    qb, kb, vb, bt, sl = _meta_inputs(dtype=torch.bfloat16)
    mask = torch.empty(3, 8, 1, dtype=torch.int32, device="meta")
    out = torch.ops.sqa.paged_attention_planned(qb, kb, vb, bt, sl, mask, 0.088, 1.0, 3000)
    assert out.shape == qb.shape and out.dtype == torch.bfloat16
    out = torch.ops.sqa.paged_attention_planned(qb, kb, vb, bt, sl, None, 0.088, 1.0, 0)
    assert out.shape == qb.shape
