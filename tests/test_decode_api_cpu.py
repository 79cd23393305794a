"""CPU checks of the FlashInfer-shaped API's argument handling (no kernel launches).

Contract violations raise ``ValueError`` before anything touches a GPU.
"""

import pytest
import torch

from small_q_attention_amd import decode_api as fi


def _args(layout="NHD"):
    q = torch.zeros(4 * 2, 32, 128, dtype=torch.float16)
    if layout == "NHD":
        kv = torch.zeros(6, 2, 16, 8, 128, dtype=torch.float16)
    else:
        kv = torch.zeros(6, 2, 8, 16, 128, dtype=torch.float16)
    bt = torch.zeros(2, 3, dtype=torch.int32)
    sl = torch.tensor([40, 20], dtype=torch.int32)
    return q, kv, None, bt, sl, 40, 128 ** -0.5, 1.0


def test_views_of_interleaved_caches():
    q, kv, *_ = _args("NHD")
    k, v = fi._kv_views(kv, "NHD")
    assert k.shape == (6, 16, 8, 128) and k.data_ptr() == kv.data_ptr()
    assert v.data_ptr() == kv[:, 1].data_ptr() and k.stride() == v.stride() == kv[:, 0].stride()
    q, kv, *_ = _args("HND")
    k, v = fi._kv_views(kv, "HND")
    assert k.shape == (6, 16, 8, 128) and k.stride() == (2 * 8 * 16 * 128, 128, 16 * 128, 1)
    with pytest.raises(ValueError, match="kv_layout"):
        fi._kv_views(kv, "NDH")
    with pytest.raises(ValueError, match="kv_cache"):
        fi._kv_views(kv[:, 0], "NHD")


@pytest.mark.parametrize("kw,match", [
    (dict(window_left=128), "window"),
    (dict(sinks=torch.zeros(32)), "sinks"),
    (dict(kv_layout="XYZ"), "kv_layout"),
    (dict(), "GPU tensors"),
])
def test_xqa_rejects_what_it_does_not_support(kw, match):
    with pytest.raises(ValueError, match=match):
        fi.xqa_batch_decode_with_kv_cache(*_args(), q_len_per_req=4, **kw)


def test_wrappers_reject_unsupported_plans():
    indptr = torch.tensor([0, 2, 3], dtype=torch.int32)
    ids = torch.tensor([4, 1, 2], dtype=torch.int32)
    last = torch.tensor([3, 16], dtype=torch.int32)
    dec = fi.BatchDecodeWithPagedKVCacheWrapper(None, "NHD")
    with pytest.raises(RuntimeError, match="plan"):
        dec.run(torch.zeros(2, 32, 128), torch.zeros(3, 2, 16, 8, 128))
    for kw, match in ((dict(pos_encoding_mode="ROPE_LLAMA"), "pos_encoding"),
                      (dict(logits_soft_cap=30.0), "soft"),
                      (dict(window_left=64), "window"),
                      (dict(q_data_type=torch.float32), "fp16 or bf16")):
        with pytest.raises(ValueError, match=match):
            dec.plan(indptr, ids, last, 32, 8, 128, 16, **kw)
    with pytest.raises(ValueError, match="head_dim"):
        dec.plan(indptr, ids, last, 32, 8, 96, 16)
    pre = fi.BatchPrefillWithPagedKVCacheWrapper(None, "HND")
    with pytest.raises(ValueError, match="same query length"):
        pre.plan(torch.tensor([0, 2, 5], dtype=torch.int32), indptr, ids, last, 32, 8, 128, 16)
    with pytest.raises(ValueError, match="custom"):
        pre.plan(torch.tensor([0, 2, 4], dtype=torch.int32), indptr, ids, last, 32, 8, 128, 16,
                 custom_mask=torch.ones(8, dtype=torch.bool))
    with pytest.raises(ValueError, match="kv_layout"):
        fi.BatchPrefillWithPagedKVCacheWrapper(None, "NDH")


@pytest.mark.parametrize("call,match", [
    (lambda w, q, kv: w.run(q, kv, None), "positionally"),
    (lambda w, q, kv: w.run(q, kv, return_lse=True), "lse"),
    (lambda w, q, kv: w.run(q, kv, lse=torch.zeros(1)), "lse"),
    (lambda w, q, kv: w.run(q, kv, window_left=128), "window"),
    (lambda w, q, kv: w.run(q, kv, sinks=torch.zeros(32)), "sinks"),
    (lambda w, q, kv: w.run(q, kv, logits_soft_cap=30.0), "unsupported run"),
])
def test_wrapper_run_rejects_what_it_would_otherwise_drop(call, match):
    """FlashInfer run() arguments this build cannot honour raise instead of being ignored
    (checked before the plan and before any tensor reaches the library)."""
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    kv = torch.zeros(3, 2, 16, 8, 128, dtype=torch.float16)
    for cls in (fi.BatchDecodeWithPagedKVCacheWrapper, fi.BatchPrefillWithPagedKVCacheWrapper):
        with pytest.raises(ValueError, match=match):
            call(cls(None, "NHD"), q, kv)


def test_run_checks_every_pointer_argument_for_the_device():
    """The shared launch refuses host tensors for each raw-pointer argument (the GPU
    tests repeat this on a real device with the rest of the call valid)."""
    q, kv, _, bt, sl, msl, s1, s2 = _args()
    with pytest.raises(ValueError, match="GPU"):
        fi.xqa_batch_decode_with_kv_cache(q, kv, None, bt, sl, msl, s1, s2, q_len_per_req=4)
