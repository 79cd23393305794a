"""CPU checks that pin the oracle's draft-mask, scale and cache-layout extensions.

The packed speculative-decoding mask follows the reference's FlashInfer
comparison scripts (``/root/reference/scripts/run_flashinfer_baseline.py:56-85``):
32-bit little-endian words stored as uint16 pairs, bit j = draft token j. Each
extension is checked against something independent of its own code path: known
bit patterns, the unmasked oracle (causal and "full" masks reduce to it), a
per-row brute force that gathers the visible tokens explicitly, linearity of the
scales, and the separate-cache oracle for the interleaved layouts.
"""

import numpy as np
import pytest
import torch

from oracle import attention_c64, attention_numpy
from oracle.vectorized import unpack_draft_mask
from small_q_attention_amd import inputs
from small_q_attention_amd.decode_api import csr_to_block_table
from small_q_attention_amd.masks import as_words, pack_draft_mask, spec_dec_mask


def _case(lens, q_len, seed, hkv=8):
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=seed, num_kv_heads=hkv)
    return inputs.make_inputs(c)


def test_packing_known_answers():
    # causal: row qi holds bits 0..qi; uint16 pairs are (low half, high half).
    m = spec_dec_mask(1, 2)
    assert m.dtype == torch.uint16 and m.shape == (1, 2, 2)
    assert m[0].tolist() == [[1, 0], [3, 0]]
    m = spec_dec_mask(2, 4)
    assert as_words(m, 2, 4)[1].flatten().tolist() == [1, 3, 7, 15]
    m = spec_dec_mask(1, 16, "full")
    assert m[0, 5].tolist() == [0xFFFF, 0]
    # 17 draft tokens still fit one word: the last row spills into the high half.
    m = spec_dec_mask(1, 17)
    assert m[0, 16].tolist() == [0xFFFF, 1]
    # 33 tokens need a second word.
    m = spec_dec_mask(1, 33)
    assert m.shape == (1, 33, 4) and m[0, 32].tolist() == [0xFFFF, 0xFFFF, 1, 0]
    with pytest.raises(ValueError):
        spec_dec_mask(1, 4, "tree")


@pytest.mark.parametrize("q_len", [1, 2, 5, 16, 33, 64])
def test_packer_and_oracle_unpacker_round_trip(q_len):
    g = torch.Generator().manual_seed(q_len)
    vis = torch.rand(3, q_len, q_len, generator=g) < 0.5
    packed = pack_draft_mask(vis)
    assert np.array_equal(unpack_draft_mask(packed, q_len), vis.numpy())
    words = as_words(packed, 3, q_len)
    assert np.array_equal(unpack_draft_mask(words, q_len), vis.numpy())


@pytest.mark.parametrize("q_len", [2, 8, 16])
def test_causal_mask_is_the_default_chain(q_len):
    q, k, v, bt, sl = _case([q_len - 1, q_len, 40, 77], q_len, seed=q_len)
    mask = spec_dec_mask(4, q_len)
    base_np = attention_numpy(q, k, v, bt, sl, 16, 8)
    assert np.array_equal(attention_numpy(q, k, v, bt, sl, 16, 8, draft_mask=mask), base_np)
    base_c = attention_c64(q, k, v, bt, sl, 16, 8)
    assert np.array_equal(attention_c64(q, k, v, bt, sl, 16, 8, draft_mask=mask), base_c)


def test_full_mask_rows_see_the_whole_sequence():
    """With every draft bit set, row qi attends to all L tokens: the unmasked oracle
    run with that row alone as a 1-token draft."""
    q_len, lens = 4, [9, 40]
    q, k, v, bt, sl = _case(lens, q_len, seed=3)
    full = attention_c64(q, k, v, bt, sl, 16, 8, draft_mask=spec_dec_mask(2, q_len, "full"))
    for qi in range(q_len):
        one = attention_c64(q[:, qi:qi + 1].contiguous(), k, v, bt, sl, 16, 8)
        assert np.allclose(full[:, qi], one[:, 0], rtol=0, atol=1e-13)


def _brute_row(q_row, k, v, bt_row, length, kvh, visible_tokens, scale):
    """Explicit gather of the visible tokens, softmax, weighted V (float64)."""
    ks = np.stack([k[bt_row[t // 16], t % 16, kvh] for t in visible_tokens]).astype(np.float64)
    vs = np.stack([v[bt_row[t // 16], t % 16, kvh] for t in visible_tokens]).astype(np.float64)
    s = ks @ q_row.astype(np.float64) * scale
    w = np.exp(s - s.max())
    return (w[:, None] * vs).sum(0) / w.sum()


def test_tree_mask_against_brute_force():
    q_len, lens = 5, [5, 23, 50]
    q, k, v, bt, sl = _case(lens, q_len, seed=5)
    g = torch.Generator().manual_seed(11)
    vis = torch.rand(3, q_len, q_len, generator=g) < 0.5
    vis[:, torch.arange(q_len), torch.arange(q_len)] = True  # a draft token sees itself
    mask = pack_draft_mask(vis)
    got_c = attention_c64(q, k, v, bt, sl, 16, 8, draft_mask=mask)
    got_np = attention_numpy(q, k, v, bt, sl, 16, 8, draft_mask=mask)
    assert np.allclose(got_c, got_np, rtol=0, atol=1e-12)
    qn, kn, vn, btn = q.numpy(), k.numpy(), v.numpy(), bt.numpy()
    for b, length in enumerate(lens):
        base = length - q_len
        for qi in range(q_len):
            tokens = [t for t in range(length)
                      if t < base or vis[b, qi, t - base]]
            for h in (0, 5, 31):
                ref = _brute_row(qn[b, qi, h], kn, vn, btn[b], length, h // 4, tokens, 128 ** -0.5)
                assert np.allclose(got_c[b, qi, h], ref, rtol=0, atol=1e-12)


def test_rows_that_see_nothing_are_zero():
    q_len = 4
    q, k, v, bt, sl = _case([2, 30], q_len, seed=6)
    vis = torch.zeros(2, q_len, q_len, dtype=torch.bool)
    out = attention_c64(q, k, v, bt, sl, 16, 8, draft_mask=pack_draft_mask(vis))
    # Sequence 0 (2 tokens, both in the draft block) sees nothing; sequence 1 only its prefix.
    assert np.all(out[0] == 0)
    # A 1-token draft over the first L - Q tokens sees exactly that prefix.
    prefix = attention_c64(q[1:, 3:4].contiguous(), k, v, bt[1:], sl[1:] - q_len, 16, 8)
    assert np.allclose(out[1, 3], prefix[0, 0], rtol=0, atol=1e-13)


def test_scales_are_linear():
    q_len = 8
    q, k, v, bt, sl = _case([100, 33], q_len, seed=7)
    s = 0.05
    scaled = attention_numpy(q, k, v, bt, sl, 16, 8, scale=s)
    via_q = attention_numpy(q.double().numpy() * (s / 128 ** -0.5), k, v, bt, sl, 16, 8)
    assert np.allclose(scaled, via_q, rtol=1e-12, atol=1e-13)
    c = attention_c64(q, k, v, bt, sl, 16, 8, scale=s, out_scale=0.25)
    assert np.allclose(c, 0.25 * scaled, rtol=1e-12, atol=1e-13)


def test_interleaved_layouts_read_in_place():
    """NHD [P, 2, 16, Hkv, D] and HND [P, 2, Hkv, 16, D] caches hold the same pages;
    the oracle reads their halves through strides and must match the separate caches."""
    q, k, v, bt, sl = _case([70, 16, 5], 4, seed=8)
    base = attention_c64(q, k, v, bt, sl, 16, 8)
    nhd = torch.stack([k, v], dim=1)
    hnd = nhd.permute(0, 1, 3, 2, 4).contiguous()
    for kk, vv in ((nhd[:, 0], nhd[:, 1]), (hnd[:, 0].transpose(1, 2), hnd[:, 1].transpose(1, 2))):
        assert not kk.is_contiguous()
        assert np.array_equal(attention_c64(q, kk, vv, bt, sl, 16, 8), base)
        assert np.allclose(attention_numpy(q, kk, vv, bt, sl, 16, 8), base, rtol=0, atol=1e-12)


def test_csr_to_block_table():
    indptr = torch.tensor([0, 3, 3, 4, 9], dtype=torch.int32)
    indices = torch.tensor([7, 2, 9, 4, 1, 1, 0, 8, 3], dtype=torch.int32)
    last = torch.tensor([5, 16, 16, 1], dtype=torch.int32)
    bt, sl = csr_to_block_table(indptr, indices, last)
    assert bt.dtype == torch.int32 and sl.dtype == torch.int32
    assert bt.tolist() == [[7, 2, 9, 0, 0], [0, 0, 0, 0, 0], [4, 0, 0, 0, 0], [1, 1, 0, 8, 3]]
    assert sl.tolist() == [2 * 16 + 5, 0, 16, 4 * 16 + 1]
    with pytest.raises(ValueError):
        csr_to_block_table(indptr, indices, torch.tensor([0, 16, 16, 1], dtype=torch.int32))
    with pytest.raises(ValueError):
        csr_to_block_table(torch.tensor([0, 3, 2], dtype=torch.int32), indices[:3],
                           torch.tensor([1, 1], dtype=torch.int32))


def test_bf16_decoding_matches_torch_on_every_pattern():
    from oracle.cbrute import _load

    lib = _load()
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    want = bits.view(torch.bfloat16).double().numpy()
    got = np.array([lib.sqa_oracle_bf16_to_double(i) for i in range(65536)])
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def _bf16_case(lens, q_len, seed, exact_in_fp16=False):
    q, k, v, bt, sl = _case(lens, q_len, seed)
    if exact_in_fp16:
        # Multiples of 1/8 in [-4, 4]: exactly representable in fp16 and in bf16.
        q, k, v = ((t.float() * 8).round().clamp(-32, 32) / 8 for t in (q, k, v))
    return q.bfloat16(), k.bfloat16(), v.bfloat16(), bt, sl


def test_bf16_oracles_agree():
    q, k, v, bt, sl = _bf16_case([9, 40, 300], 4, seed=21)
    c = attention_c64(q, k, v, bt, sl, 16, 8)
    n = attention_numpy(q, k, v, bt, sl, 16, 8)
    assert np.allclose(c, n, rtol=0, atol=1e-12)
    mask = spec_dec_mask(3, 4, "full")
    c = attention_c64(q, k, v, bt, sl, 16, 8, draft_mask=mask)
    n = attention_numpy(q, k, v, bt, sl, 16, 8, draft_mask=mask)
    assert np.allclose(c, n, rtol=0, atol=1e-12)


def test_bf16_and_fp16_paths_agree_on_shared_values():
    """Values representable in both types: the bf16 and fp16 decodings must give the
    same float64 result bit for bit."""
    q, k, v, bt, sl = _bf16_case([33, 200], 8, seed=22, exact_in_fp16=True)
    as_bf16 = attention_c64(q, k, v, bt, sl, 16, 8)
    as_fp16 = attention_c64(q.half(), k.half(), v.half(), bt, sl, 16, 8)
    assert np.array_equal(as_bf16, as_fp16)
    with pytest.raises(ValueError, match="element type"):
        attention_c64(q, k.half(), v.half(), bt, sl, 16, 8)


def test_fp8_decoding_matches_torch_on_every_pattern():
    from oracle.cbrute import _load

    lib = _load()
    want = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn)
    want = want.double().numpy()
    got = np.array([lib.sqa_oracle_fp8_to_double(i) for i in range(256)])
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and np.isnan(got[0x7F])


def _fp8_case(lens, q_len, seed):
    q, k, v, bt, sl = _case(lens, q_len, seed)
    return q, k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn), bt, sl


def test_fp8_cache_oracle():
    """e4m3 caches: every e4m3 value is exact in fp16, so the oracle on the e4m3 bytes
    equals the oracle on the same values stored as fp16 (bit for bit), for fp16 and
    bf16 queries; the numpy restatement agrees."""
    q, k8, v8, bt, sl = _fp8_case([9, 70, 300], 8, seed=31)
    k16, v16 = k8.to(torch.float16), v8.to(torch.float16)
    assert torch.equal(k16.to(torch.float8_e4m3fn).view(torch.uint8), k8.view(torch.uint8))
    a = attention_c64(q, k8, v8, bt, sl, 16, 8)
    assert np.array_equal(a, attention_c64(q, k16, v16, bt, sl, 16, 8))
    assert np.allclose(a, attention_numpy(q, k8, v8, bt, sl, 16, 8), rtol=0, atol=1e-12)
    qb = q.bfloat16()
    ab = attention_c64(qb, k8, v8, bt, sl, 16, 8, scale=0.05, out_scale=2.0)
    assert np.array_equal(ab, attention_c64(qb, k16.bfloat16(), v16.bfloat16(), bt, sl, 16, 8,
                                            scale=0.05, out_scale=2.0))
    # Interleaved e4m3 cache read through strides.
    kv = torch.stack([k8.view(torch.uint8), v8.view(torch.uint8)], 1).view(torch.float8_e4m3fn)
    assert np.array_equal(attention_c64(q, kv[:, 0], kv[:, 1], bt, sl, 16, 8), a)
