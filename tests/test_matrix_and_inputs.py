"""CPU checks of the 36-case matrix definition and the synthetic input generator.

The matrix test restates ``/root/reference/tests/test_matrix.py:6-17``.
"""

import itertools
import json
from pathlib import Path

import torch

from small_q_attention_amd import inputs, matrix

MATRIX = Path(matrix.__file__).resolve().parent / "configs" / "core_matrix.json"


def test_core_matrix_is_36_cases():
    config, cases = matrix.load_cases(MATRIX)
    assert len(cases) == 36
    assert config["kernel_v0_q_len"] == [2, 4, 8]
    assert config["supported_q_len"] == [2, 4, 8, 16]
    assert {c["q_len"] for c in cases} == {2, 4, 8, 16}


def test_matrix_contract_is_fixed():
    config, _ = matrix.load_cases(MATRIX)
    assert config["dtype"] == "float16"
    assert config["head_dim"] == 128
    assert config["page_size"] == 16
    assert (config["num_query_heads"], config["num_kv_heads"]) == (32, 8)


def test_matrix_cases_match_the_product():
    config = json.loads(MATRIX.read_text())
    expect = list(itertools.product(config["q_len"], config["kv_len"], config["batch_size"]))
    got = [(c.q_len, c.seq_lens[0], c.batch) for c in inputs.matrix_cases()]
    assert got == expect


def test_generator_is_deterministic_and_seed_sensitive():
    case = inputs.Case(batch=2, q_len=4, seq_lens=[40, 17], seed=5)
    a = inputs.make_inputs(case)
    b = inputs.make_inputs(case)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    c = inputs.make_inputs(inputs.Case(batch=2, q_len=4, seq_lens=[40, 17], seed=6))
    assert not torch.equal(a[0], c[0])


def test_random_page_table_is_a_disjoint_draw_from_a_2x_pool():
    case = inputs.Case(batch=3, q_len=2, seq_lens=[33, 16, 100], seed=7)
    q, k, v, bt, sl = inputs.make_inputs(case)
    pages = case.pages_per_seq
    assert pages == [3, 1, 7]
    assert k.shape[0] == 2 * sum(pages)
    used = torch.cat([bt[b, :n] for b, n in enumerate(pages)])
    assert used.unique().numel() == used.numel()  # no page shared between sequences
    assert int(used.min()) >= 0 and int(used.max()) < k.shape[0]
    assert sl.tolist() == [33, 16, 100]
    assert bt.dtype == torch.int32 and sl.dtype == torch.int32
    assert q.dtype == k.dtype == v.dtype == torch.float16


def test_shared_and_unique_modes_reverse_page_ids():
    """The reference runner's page modes (scripts/run_gpu_matrix.py:42-48)."""
    shared = inputs.Case(batch=2, q_len=2, seq_lens=[48, 48], page_mode="shared")
    _, k, _, bt, _ = inputs.make_inputs(shared)
    assert bt.tolist() == [[2, 1, 0], [2, 1, 0]] and k.shape[0] == 3
    unique = inputs.Case(batch=2, q_len=2, seq_lens=[48, 48], page_mode="unique")
    _, k, _, bt, _ = inputs.make_inputs(unique)
    assert bt.tolist() == [[2, 1, 0], [5, 4, 3]] and k.shape[0] == 6


def test_outliers_scale_about_the_requested_fraction():
    case = inputs.Case(batch=1, q_len=2, seq_lens=[4096], seed=9, k_outlier_frac=0.01)
    plain = inputs.Case(batch=1, q_len=2, seq_lens=[4096], seed=9)
    k1 = inputs.make_inputs(case)[1].float()
    k0 = inputs.make_inputs(plain)[1].float()
    scaled = (k1 != k0).flatten(2).any(-1)  # [pages, slots]
    frac = scaled.float().mean().item()
    assert 0.005 < frac < 0.015
    # x4 is exact in fp16 except for subnormals, hence the small atol.
    assert torch.allclose(k1[scaled], 4.0 * k0[scaled], atol=1e-3, rtol=0)
    assert torch.equal(k1[~scaled], k0[~scaled])


def test_ragged_lengths_in_range_and_byte_counts():
    case = inputs.ragged_case(16, 8, 1024, 32768, seed=5)
    assert all(1024 <= n <= 32768 for n in case.seq_lens)
    assert len(set(case.seq_lens)) > 8
    assert inputs.kv_bytes([32768] * 16) == 2147483648
    cfg3 = inputs.baseline_configs()["cfg3"]
    assert inputs.kv_bytes(cfg3.seq_lens) == 16 * 32768 * 8 * 128 * 2 * 2
    assert inputs.attention_flops(cfg3) == 4 * 32 * 128 * 16 * sum(32768 - 8 + i + 1 for i in range(8))


def test_runner_defaults_are_the_reference_runners():
    """An invocation relying on the defaults measures the reference runner's workload
    (``/root/reference/scripts/run_gpu_matrix.py:111-127``): variants v0 v1, shared
    pages, integer chunk_keys 512, q_len 2 4 8, KV 1024 8192, batch 1 4, warmup 5,
    repeats 15, 3 cases checked; ``auto`` and ``random`` stay opt-ins."""
    args = matrix.build_parser().parse_args([])
    assert args.variants == ["v0", "v1"]
    assert args.page_mode == "shared"
    assert args.chunk_keys == 512 and isinstance(args.chunk_keys, int)
    assert args.token_group == 2
    assert args.q_lens == [2, 4, 8] and args.kv_lens == [1024, 8192]
    assert args.batch_sizes == [1, 4]
    assert (args.warmup, args.repeats, args.limit) == (5, 15, 0)
    assert not args.check_correctness and args.correctness_limit == 3
    opt = matrix.build_parser().parse_args(["--variants", "auto", "v3", "--chunk-keys", "auto",
                                            "--page-mode", "random"])
    assert opt.variants == ["auto", "v3"] and opt.chunk_keys == "auto"
    assert opt.page_mode == "random"
    assert matrix.build_parser().parse_args(["--chunk-keys", "128"]).chunk_keys == 128
    import pytest

    with pytest.raises(SystemExit):
        matrix.build_parser().parse_args(["--chunk-keys", "lots"])
