"""CPU pins of the two checkers the parity suite leans on besides the C oracle.

* ``small_q_attention_amd.checker.attention_fp32`` (``tests/_helpers.torch_fp32_reference``):
  the float32 torch statement the full-size GPU tests and the matrix runner's
  ``--check-correctness`` compare against. Here it must agree with the float64 C
  oracle (``oracle.attention_c64``) on ragged, partial-page, q_len-16, GQA and
  short-row cases (``seq_len < q_len``, where rows that see no key are 0).
* The fp16-input branch of the loop-faithful oracle
  (``/root/reference/src/small_q_attention/reference.py:68-70``: fp16 logits,
  fp32 softmax cast back to fp16, fp16 PV). Closed forms where every
  probability and product is exact in fp16 must give the fp32 branch's result
  rounded to fp16, bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import attention_c64, paged_mtp_attention_reference
from small_q_attention_amd import inputs
from small_q_attention_amd.checker import attention_fp32

CASES = [
    # (label, batch, q_len, seq_lens, hq, hkv, head_dim)
    ("ragged_partial_pages", 4, 8, [33, 1000, 17, 250], 32, 8, 128),
    ("q16_spans_pages", 2, 16, [16, 49], 32, 8, 128),
    ("short_rows", 3, 8, [3, 8, 9], 32, 8, 128),          # rows with no key, and seq_len == q_len
    ("mha_and_mqa", 2, 4, [21, 64], 8, 8, 64),
    ("mqa", 2, 2, [40, 7], 8, 1, 64),
    ("contract_shape", 2, 4, [1024, 531], 32, 8, 128),
]


@pytest.mark.parametrize("label,batch,q_len,lens,hq,hkv,dim", CASES, ids=[c[0] for c in CASES])
def test_fp32_checker_matches_the_float64_oracle(label, batch, q_len, lens, hq, hkv, dim):
    case = inputs.Case(batch=batch, q_len=q_len, seq_lens=lens, num_query_heads=hq,
                       num_kv_heads=hkv, head_dim=dim, seed=11, k_outlier_frac=0.05)
    q, k, v, bt, sl = inputs.make_inputs(case)
    ref = attention_c64(q, k, v, bt, sl, case.page_size, hkv)
    got = attention_fp32(q, k, v, bt, sl, case.page_size, hkv)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5)
    # Rows that see no key (seq_len - q_len + qi + 1 <= 0) are exactly 0 in both.
    for b, n in enumerate(lens):
        for qi in range(q_len):
            if n - q_len + qi + 1 <= 0:
                assert not np.any(got[b, qi]) and not np.any(ref[b, qi])


def test_fp32_checker_sees_a_planted_mask_error():
    """The comparison above is tight enough to catch an off-by-one visible count."""
    case = inputs.Case(batch=1, q_len=4, seq_lens=[20], seed=3)
    q, k, v, bt, sl = inputs.make_inputs(case)
    ref = attention_c64(q, k, v, bt, sl, 16, 8)
    # One token fewer visible per row = the checker run on a sequence one shorter
    # with the draft block shifted back by one.
    shifted = attention_fp32(q, k, v, bt, sl - 1, 16, 8)
    assert np.abs(shifted - ref).max() > 1e-3


def _tiny(q, k, v, lens, q_len, page=4, hkv=1):
    """fp16 tensors -> (query, key_cache, value_cache, block_tables, seq_lens) with the
    tokens of every sequence stored in order on consecutive pages."""
    batch = len(lens)
    pages = [-(-n // page) for n in lens]
    bt = torch.zeros(batch, max(pages), dtype=torch.int32)
    off = 0
    for b, p in enumerate(pages):
        bt[b, :p] = torch.arange(off, off + p, dtype=torch.int32)
        off += p
    return q, k, v, bt, torch.tensor(lens, dtype=torch.int32)


def _both_branches(args, page=4, hkv=1):
    q, k, v, bt, sl = args
    out16 = paged_mtp_attention_reference(q, k, v, bt, sl, page, hkv)
    out32 = paged_mtp_attention_reference(q.float(), k.float(), v.float(), bt, sl, page, hkv)
    assert out16.dtype == torch.float16 and out32.dtype == torch.float32
    return out16, out32


def test_fp16_branch_uniform_softmax_is_exact():
    """Q = 0: every visible key weighs 1/n; with n = 4 and 8 (q_len 1) the weights, the
    integer V rows and their means are exact in fp16."""
    dim, lens = 8, [4, 8]
    g = torch.Generator().manual_seed(5)
    k = torch.randn(3, 4, 1, dim, generator=g).half()
    v = torch.randint(-8, 9, (3, 4, 1, dim), generator=g).half()
    q = torch.zeros(2, 1, 2, dim, dtype=torch.float16)
    out16, out32 = _both_branches(_tiny(q, k, v, lens, 1))
    toks = v.reshape(-1, dim).double()
    expect = torch.stack([toks[:4].mean(0), toks[4:12].mean(0)])  # sequence 1 = pages 1, 2
    for b in range(2):
        for h in range(2):
            assert torch.equal(out16[b, 0, h].double(), expect[b])
    assert torch.equal(out16, out32.half())


def test_fp16_branch_three_to_one_weights():
    """Logits ln 3 (rounded to fp16) and 0 give weights 0.750004 / 0.249996 in fp32,
    which the fp16 branch rounds to exactly 3/4 and 1/4: V rows 4 and 8 give 5."""
    dim = 4  # scale 1/2
    ln3 = torch.tensor(np.log(3.0)).half()
    q = torch.zeros(1, 1, 1, dim, dtype=torch.float16)
    q[0, 0, 0, 0] = 2.0  # (k . q) * 1/2 = k[0]
    k = torch.zeros(1, 4, 1, dim, dtype=torch.float16)
    k[0, 0, 0, 0] = ln3
    v = torch.zeros(1, 4, 1, dim, dtype=torch.float16)
    v[0, 0, 0, :] = 4.0
    v[0, 1, 0, :] = 8.0
    out16, out32 = _both_branches(_tiny(q, k, v, [2], 1))
    assert torch.all(out16 == 5.0)
    assert not torch.all(out32 == 5.0)  # the fp32 branch keeps the unrounded weights
    assert torch.equal(out16, out32.half())


def test_fp16_branch_dominant_key_selects_its_row():
    """A logit 24 above the rest gives weight 1 - 4e-11 -> exactly 1.0 in fp16 (the rest
    round to 0): each row returns the V row of its dominant key, in page order."""
    dim, page = 8, 4
    lens, q_len = [7], 2  # rows see 6 and 7 keys
    q = torch.zeros(1, q_len, 1, dim, dtype=torch.float16)
    q[0, :, 0, 0] = 8.0
    k = torch.zeros(2, page, 1, dim, dtype=torch.float16)
    v = torch.randint(-8, 9, (2, page, 1, dim), generator=torch.Generator().manual_seed(1)).half()
    # Physical pages in reverse order: token t lives on page 1 - t // 4.
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    kt = k.view(2, page, dim)
    kt[1, 3, 0] = 12.0  # token 3 -> logit 8 * 12 / sqrt(8) = 33.9 for both rows
    q_, k_, v_, _, sl = _tiny(q, k, v, lens, q_len)
    out16, out32 = _both_branches((q_, k_, v_, bt, sl))
    for qi in range(q_len):
        assert torch.equal(out16[0, qi, 0], v.view(2, page, dim)[1, 3])
    assert torch.equal(out16, out32.half())
