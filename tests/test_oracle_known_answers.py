"""Pins the CPU oracle (``oracle/``) before it is trusted as the checker.

Each test fixes a property a plausible mistake in a restatement would break:
the reference's own known-answer tests (restated, with the zero fixture
corrected), closed forms, invariants, and agreement of three independently
written restatements (torch loop, numpy vectorized, C double brute force).
Reference tests restated: ``/root/reference/tests/test_reference.py:9-45`` and
``/root/reference/tests/test_reference_edges.py:17-78``.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import attention_c64, attention_numpy, paged_mtp_attention_reference


def _single_head_softmax(keys, values, q, scale):
    """Plain softmax attention of one query over a key list (float64 numpy)."""
    s = keys @ q * scale
    w = np.exp(s - s.max())
    return (w / w.sum()) @ values


def _all_oracles(q, k, v, bt, sl, page, hkv):
    loop = paged_mtp_attention_reference(q.float(), k.float(), v.float(), bt, sl, page, hkv)
    vec = attention_numpy(q, k, v, bt, sl, page, hkv)
    return loop.double().numpy(), vec


# --- reference tests restated -------------------------------------------------

def test_manual_single_head_case():
    """reference tests/test_reference.py:9-32: one kv head, two query heads, page 2."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 2, 2, 4, generator=g)
    kc = torch.randn(2, 2, 1, 4, generator=g)
    vc = torch.randn(2, 2, 1, 4, generator=g)
    bt = torch.tensor([[0, 1]], dtype=torch.int32)
    sl = torch.tensor([4], dtype=torch.int32)
    out = paged_mtp_attention_reference(q, kc, vc, bt, sl, page_size=2, num_kv_heads=1)
    keys = kc.reshape(4, 4).double().numpy()
    vals = vc.reshape(4, 4).double().numpy()
    for qi in range(2):
        visible = 4 - 2 + qi + 1
        for qh in range(2):
            exp = _single_head_softmax(keys[:visible], vals[:visible], q[0, qi, qh].double().numpy(), 0.5)
            np.testing.assert_allclose(out[0, qi, qh].double().numpy(), exp, rtol=1e-5, atol=1e-6)


def test_gqa_output_shape():
    """reference tests/test_reference.py:35-45 (Hq/Hkv = 4/2)."""
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 2, 4, 8, generator=g)
    kc = torch.randn(2, 4, 2, 8, generator=g)
    vc = torch.randn(2, 4, 2, 8, generator=g)
    out = paged_mtp_attention_reference(q, kc, vc, torch.tensor([[0, 1]], dtype=torch.int32),
                                        torch.tensor([5], dtype=torch.int32), 4, 2)
    assert out.shape == q.shape


def test_physical_page_order_is_honoured():
    """reference tests/test_reference_edges.py:17-31: block table [2, 0, 1], seq_len 5."""
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 2, 2, 4, generator=g)
    kc = torch.randn(3, 2, 1, 4, generator=g)
    vc = torch.randn(3, 2, 1, 4, generator=g)
    bt = torch.tensor([[2, 0, 1]], dtype=torch.int32)
    out = paged_mtp_attention_reference(q, kc, vc, bt, torch.tensor([5], dtype=torch.int32), 2, 1)
    # Logical token order: page 2 slots 0,1; page 0 slots 0,1; page 1 slot 0.
    order = [(2, 0), (2, 1), (0, 0), (0, 1), (1, 0)]
    keys = np.stack([kc[p, s, 0].double().numpy() for p, s in order])
    vals = np.stack([vc[p, s, 0].double().numpy() for p, s in order])
    for qi in range(2):
        visible = 5 - 2 + qi + 1
        for qh in range(2):
            exp = _single_head_softmax(keys[:visible], vals[:visible], q[0, qi, qh].double().numpy(), 0.5)
            np.testing.assert_allclose(out[0, qi, qh].double().numpy(), exp, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("seq_lens", [[1], [4, 4]])
def test_invalid_metadata_raises(seq_lens):
    """reference tests/test_reference_edges.py:34-52: seq_len < q_len, batch mismatch."""
    q = torch.randn(1, 2, 2, 4)
    kc = torch.randn(3, 2, 1, 4)
    vc = torch.randn(3, 2, 1, 4)
    bt = torch.tensor([[2, 0, 1]], dtype=torch.int32)
    with pytest.raises(ValueError):
        paged_mtp_attention_reference(q, kc, vc, bt, torch.tensor(seq_lens, dtype=torch.int32), 2, 1)


@pytest.mark.parametrize("case", ["ndim", "divisible", "kshape", "vshape"])
def test_contract_violations_raise(case):
    """reference.py:34-44: every contract check raises ValueError."""
    q = torch.randn(1, 2, 4, 8)
    kc = torch.randn(2, 4, 2, 8)
    vc = torch.randn(2, 4, 2, 8)
    bt = torch.tensor([[0, 1]], dtype=torch.int32)
    sl = torch.tensor([5], dtype=torch.int32)
    kw = dict(page_size=4, num_kv_heads=2)
    if case == "ndim":
        q = q[0]
    elif case == "divisible":
        kw["num_kv_heads"] = 3
    elif case == "kshape":
        kw["page_size"] = 2
    else:
        vc = torch.randn(2, 4, 2, 4)
    with pytest.raises(ValueError):
        paged_mtp_attention_reference(q, kc, vc, bt, sl, **kw)


def test_zero_fixture_gives_mean_of_visible_values():
    """reference tests/test_reference_edges.py:55-66, corrected.

    The reference fixture reshapes arange(8) to (2, 2, 1, 4), which needs 16
    elements, and expects rows 0/1 to average V[:1] / V[:2]. With seq_len 4 and
    q_len 2 the visible counts are 3 and 4, so a uniform softmax (Q = K = 0)
    gives the mean of V[0:3] and of V[0:4].
    """
    q = torch.zeros(1, 2, 2, 4)
    kc = torch.zeros(2, 2, 1, 4)
    vc = torch.arange(16, dtype=torch.float32).reshape(2, 2, 1, 4)
    out = paged_mtp_attention_reference(q, kc, vc, torch.tensor([[0, 1]], dtype=torch.int32),
                                        torch.tensor([4], dtype=torch.int32), 2, 1)
    vals = vc.reshape(4, 4)
    torch.testing.assert_close(out[0, 0], vals[:3].mean(0).expand(2, 4))
    torch.testing.assert_close(out[0, 1], vals[:4].mean(0).expand(2, 4))


def test_high_magnitude_fixture_stays_finite():
    """reference tests/test_reference_edges.py:69-78: Q = K = 100, V = 1 -> ones."""
    q = torch.full((1, 2, 2, 4), 100.0)
    kc = torch.full((2, 2, 1, 4), 100.0)
    vc = torch.ones_like(kc)
    out = paged_mtp_attention_reference(q, kc, vc, torch.tensor([[0, 1]], dtype=torch.int32),
                                        torch.tensor([4], dtype=torch.int32), 2, 1)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out, torch.ones_like(out))


# --- closed forms and invariants ---------------------------------------------

def _rand_case(seed, batch=2, q_len=4, hq=8, hkv=2, dim=16, page=4, lens=(13, 9), pool=12):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, q_len, hq, dim, generator=g).half()
    kc = torch.randn(pool, page, hkv, dim, generator=g).half()
    vc = torch.randn(pool, page, hkv, dim, generator=g).half()
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    max_pages = max(-(-n // page) for n in lens)
    bt = torch.zeros(batch, max_pages, dtype=torch.int32)
    off = 0
    for b, n in enumerate(lens):
        p = -(-n // page)
        bt[b, :p] = perm[off:off + p]
        off += p
    return q, kc, vc, bt, torch.tensor(lens, dtype=torch.int32)


def test_seq_len_equal_q_len_first_row_copies_v0():
    """Row 0 sees exactly one key when seq_len == q_len, so its output is V[token 0]."""
    q, kc, vc, bt, _ = _rand_case(3, batch=1, q_len=4, lens=(4,))
    sl = torch.tensor([4], dtype=torch.int32)
    out = attention_numpy(q, kc, vc, bt, sl, 4, 2)
    pid = int(bt[0, 0])
    for qh in range(8):
        np.testing.assert_allclose(out[0, 0, qh], vc[pid, 0, qh // 4].double().numpy(), atol=1e-12)


def test_dominant_key_selects_its_value():
    """A key aligned with Q and scaled far above the rest takes all the weight."""
    q, kc, vc, bt, sl = _rand_case(4, batch=1, q_len=2, lens=(11,))
    kc = kc.float()
    q = q.float()
    target_t = 6  # visible to both rows (first row sees 11 - 2 + 1 = 10 tokens)
    pid, slot = int(bt[0, target_t // 4]), target_t % 4
    kc[pid, slot, 0] = q[0, 0, 0] * 50.0
    q[0, 1, 0] = q[0, 0, 0]
    out = attention_numpy(q, kc, vc, bt, sl, 4, 2)
    np.testing.assert_allclose(out[0, 0, 0], vc[pid, slot, 0].double().numpy(), atol=1e-9)
    np.testing.assert_allclose(out[0, 1, 0], vc[pid, slot, 0].double().numpy(), atol=1e-9)


def test_causal_boundary_is_exact():
    """Row qi depends on token L-Q+qi and not on token L-Q+qi+1 (no off-by-one)."""
    q, kc, vc, bt, sl = _rand_case(5, batch=1, q_len=4, lens=(14,))
    base = attention_numpy(q, kc, vc, bt, sl, 4, 2)
    n, ql = 14, 4
    for qi in range(ql - 1):
        t_last_visible, t_first_hidden = n - ql + qi, n - ql + qi + 1
        for t, should_change in ((t_last_visible, True), (t_first_hidden, False)):
            k2, v2 = kc.clone(), vc.clone()
            pid, slot = int(bt[0, t // 4]), t % 4
            k2[pid, slot] += 1.0
            v2[pid, slot] += 1.0
            moved = np.abs(attention_numpy(q, k2, v2, bt, sl, 4, 2)[0, qi] - base[0, qi]).max()
            assert (moved > 1e-6) == should_change, (qi, t, moved)


def test_page_table_permutation_invariance():
    """Moving pages in the pool and updating the table leaves the output unchanged."""
    q, kc, vc, bt, sl = _rand_case(6)
    base = attention_numpy(q, kc, vc, bt, sl, 4, 2)
    g = torch.Generator().manual_seed(60)
    perm = torch.randperm(kc.shape[0], generator=g)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    k2, v2 = kc[perm], vc[perm]
    bt2 = inv[bt.long()].to(torch.int32)
    np.testing.assert_allclose(attention_numpy(q, k2, v2, bt2, sl, 4, 2), base, atol=1e-12)


def test_gqa_mapping_is_floor_division():
    """Head h reads kv head h // (Hq/Hkv): changing kv head 1 moves heads 4..7 only."""
    q, kc, vc, bt, sl = _rand_case(7)
    base = attention_numpy(q, kc, vc, bt, sl, 4, 2)
    k2 = kc.clone()
    k2[:, :, 1] = torch.randn(k2[:, :, 1].shape, generator=torch.Generator().manual_seed(70)).half()
    out = attention_numpy(q, k2, vc, bt, sl, 4, 2)
    assert np.abs(out[:, :, :4] - base[:, :, :4]).max() == 0
    assert np.abs(out[:, :, 4:] - base[:, :, 4:]).max() > 1e-3


def test_scale_is_inverse_sqrt_head_dim():
    """Zero-padding D from 16 to 64 and doubling Q keeps every score, hence the output."""
    q, kc, vc, bt, sl = _rand_case(8)
    base = attention_numpy(q, kc, vc, bt, sl, 4, 2)
    pad = lambda t, n: torch.cat([t.float(), torch.zeros(*t.shape[:-1], n - t.shape[-1])], -1)  # noqa: E731
    q2, k2, v2 = pad(q, 64) * 2.0, pad(kc, 64), pad(vc, 64)
    out = attention_numpy(q2, k2, v2, bt, sl, 4, 2)[..., :16]
    np.testing.assert_allclose(out, base, atol=1e-12)


def test_uniform_softmax_is_mean_of_visible_values():
    """Q = 0 gives equal weights: row qi is the mean of its first L-Q+qi+1 values."""
    q, kc, vc, bt, sl = _rand_case(9)
    q = torch.zeros_like(q)
    out = attention_numpy(q, kc, vc, bt, sl, 4, 2)
    for b in range(2):
        n = int(sl[b])
        toks = [vc[int(bt[b, t // 4]), t % 4].double().numpy() for t in range(n)]
        toks = np.stack(toks)  # [n, Hkv, D]
        for qi in range(4):
            vis = n - 4 + qi + 1
            for qh in range(8):
                np.testing.assert_allclose(out[b, qi, qh], toks[:vis, qh // 4].mean(0), atol=1e-12)


# --- three restatements agree --------------------------------------------------

@pytest.mark.parametrize("seed,lens,q_len", [(10, (13, 9), 4), (11, (4, 17), 2), (12, (30, 5), 4)])
def test_three_oracles_agree(seed, lens, q_len):
    q, kc, vc, bt, sl = _rand_case(seed, lens=lens, q_len=q_len, pool=24)
    loop, vec = _all_oracles(q, kc, vc, bt, sl, 4, 2)
    c64 = attention_c64(q, kc, vc, bt, sl, 4, 2)
    np.testing.assert_allclose(vec, c64, atol=1e-12)
    np.testing.assert_allclose(loop, c64, atol=2e-6)


def test_three_oracles_agree_at_contract_shape():
    """Hq/Hkv 32/8, D 128, page 16, ragged lengths with partial last pages."""
    from small_q_attention_amd import inputs

    case = inputs.Case(batch=3, q_len=8, seq_lens=[33, 100, 8], seed=13)
    q, kc, vc, bt, sl = inputs.make_inputs(case)
    loop, vec = _all_oracles(q, kc, vc, bt, sl, 16, 8)
    c64 = attention_c64(q, kc, vc, bt, sl, 16, 8)
    np.testing.assert_allclose(vec, c64, atol=1e-12)
    np.testing.assert_allclose(loop, c64, atol=5e-6)


@pytest.mark.parametrize("head_dim", [64, 256])
def test_three_oracles_agree_at_other_head_dims(head_dim):
    """The head dims the kernels also build: the restatements take D from the shapes,
    and the default scale follows it (D^-1/2)."""
    from small_q_attention_amd import inputs

    case = inputs.Case(batch=2, q_len=4, seq_lens=[37, 6], seed=15, head_dim=head_dim)
    q, kc, vc, bt, sl = inputs.make_inputs(case)
    loop, vec = _all_oracles(q, kc, vc, bt, sl, 16, 8)
    c64 = attention_c64(q, kc, vc, bt, sl, 16, 8)
    np.testing.assert_allclose(vec, c64, atol=1e-12)
    np.testing.assert_allclose(loop, c64, atol=5e-6)
    explicit = attention_c64(q, kc, vc, bt, sl, 16, 8, scale=head_dim ** -0.5)
    np.testing.assert_array_equal(explicit, c64)


def test_c_oracle_rows_without_keys_are_zero_and_bad_ids_raise():
    q, kc, vc, bt, sl = _rand_case(14, batch=1, q_len=4, lens=(2,))
    out = attention_c64(q, kc, vc, bt, torch.tensor([2], dtype=torch.int32), 4, 2)
    assert np.all(out[0, :2] == 0) and np.all(np.abs(out[0, 2:]).sum(-1) > 0)
    bad = bt.clone()
    bad[0, 0] = kc.shape[0]
    with pytest.raises(IndexError):
        attention_c64(q, kc, vc, bad, torch.tensor([2], dtype=torch.int32), 4, 2)


def test_half_decoder_matches_numpy():
    """The C oracle's fp16 decoder agrees with numpy on every bit pattern class."""
    from oracle import cbrute

    lib = cbrute._load()
    bits = np.array([0, 1, 0x3ff, 0x400, 0x3c00, 0x7bff, 0x7c00, 0x8001, 0xc000, 0xfbff, 0x5555],
                    dtype=np.uint16)
    for b in bits:
        assert lib.sqa_oracle_half_to_double(int(b)) == float(b.view(np.float16))
    assert oracle.c_oracle_available()
