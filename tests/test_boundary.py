"""CPU checks of the Python op boundary (``small_q_attention_amd.cuda``).

Mirrors the reference's argument checks and their exception classes
(``/root/reference/src/small_q_attention/cuda.py:61-336``,
``csrc/small_q_attention_ext.cu:976-1002``). Device-side behaviour is in the
``gpu`` tests; here tensor stand-ins reach each check without a GPU.
"""

import inspect

import pytest
import torch

from small_q_attention_amd import cuda as sqa

CUDA0 = torch.device("cuda", 0)


class FakeTensor:
    """Just enough of a device tensor for the boundary checks."""

    def __init__(self, shape, dtype=torch.float16, is_cuda=True, contiguous=True, device=CUDA0):
        self.shape = torch.Size(shape)
        self.dtype = dtype
        self.is_cuda = is_cuda
        self._contiguous = contiguous
        self.device = device if is_cuda else torch.device("cpu")

    @property
    def ndim(self):
        return len(self.shape)

    def is_contiguous(self):
        return self._contiguous

    def numel(self):
        n = 1
        for s in self.shape:
            n *= s
        return n


def good_inputs(q_len=4, hq=32, hkv=8, dim=128, page=16):
    return dict(
        query=FakeTensor((2, q_len, hq, dim)),
        key_cache=FakeTensor((10, page, hkv, dim)),
        value_cache=FakeTensor((10, page, hkv, dim)),
        block_tables=FakeTensor((2, 5), dtype=torch.int32),
        seq_lens=FakeTensor((2,), dtype=torch.int32),
    )


FORWARDS = [sqa.forward_v0, sqa.forward_v1, sqa.forward_v2, sqa.forward_v3, sqa.forward_v4,
            sqa.forward_v5]


@pytest.fixture
def fake_gpu(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)


def _args(inp):
    return (inp["query"], inp["key_cache"], inp["value_cache"], inp["block_tables"],
            inp["seq_lens"], 16)


def test_signatures_match_the_reference():
    """Names, parameter order and defaults of reference cuda.py:61,81,120-129,177-187,238-248,297-308."""
    expect = {
        "forward_v0": ["query", "key_cache", "value_cache", "block_tables", "seq_lens",
                       "page_size", "verbose"],
        "forward_v2": ["query", "key_cache", "value_cache", "block_tables", "seq_lens",
                       "page_size", "chunk_keys", "verbose"],
        "forward_v3": ["query", "key_cache", "value_cache", "block_tables", "seq_lens",
                       "page_size", "chunk_keys", "max_seq_len", "verbose"],
        "forward_v5": ["query", "key_cache", "value_cache", "block_tables", "seq_lens",
                       "page_size", "chunk_keys", "token_group", "max_seq_len", "verbose"],
    }
    expect["forward_v1"] = expect["forward_v0"]
    expect["forward_v4"] = expect["forward_v3"]
    for name, params in expect.items():
        sig = inspect.signature(getattr(sqa, name))
        assert list(sig.parameters) == params, name
    assert inspect.signature(sqa.forward_v2).parameters["chunk_keys"].default == 512
    assert inspect.signature(sqa.forward_v3).parameters["max_seq_len"].default == 0
    assert inspect.signature(sqa.forward_v5).parameters["token_group"].default == 2
    for n in range(6):
        assert callable(getattr(sqa, f"load_v{n}"))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
@pytest.mark.parametrize("fwd", FORWARDS)
def test_no_gpu_raises_runtime_error(fwd):
    """reference cuda.py:65-66."""
    with pytest.raises(RuntimeError):
        fwd(*_args(good_inputs()))


@pytest.mark.parametrize("fwd", FORWARDS)
@pytest.mark.parametrize("mutation", ["cpu_tensor", "non_contiguous", "dtype", "q_len", "head_dim"])
def test_python_contract_raises_value_error(fake_gpu, fwd, mutation):
    """reference cuda.py:67-77 (q_len 16 is accepted here; q_len 3 is not)."""
    inp = good_inputs()
    if mutation == "cpu_tensor":
        inp["block_tables"] = FakeTensor((2, 5), dtype=torch.int32, is_cuda=False)
    elif mutation == "non_contiguous":
        inp["value_cache"] = FakeTensor((10, 16, 8, 128), contiguous=False)
    elif mutation == "dtype":
        inp["key_cache"] = FakeTensor((10, 16, 8, 128), dtype=torch.bfloat16)
    elif mutation == "q_len":
        inp["query"] = FakeTensor((2, 3, 32, 128))
    else:
        inp = good_inputs(dim=64)
    with pytest.raises(ValueError):
        fwd(*_args(inp))


@pytest.mark.parametrize("fwd", [sqa.forward_v3, sqa.forward_v4, sqa.forward_v5])
def test_gqa_group_must_be_four_for_v3_to_v5(fake_gpu, fwd):
    """reference cuda.py:208-209."""
    with pytest.raises(ValueError):
        fwd(*_args(good_inputs(hq=32, hkv=16)))


@pytest.mark.parametrize("fwd", [sqa.forward_v2, sqa.forward_v3, sqa.forward_v4, sqa.forward_v5])
def test_chunk_keys_must_be_positive(fake_gpu, fwd):
    """reference cuda.py:149-150."""
    with pytest.raises(ValueError):
        fwd(*_args(good_inputs()), 0)


def test_token_group_must_be_two_or_four(fake_gpu):
    """reference cuda.py:329-330."""
    with pytest.raises(ValueError):
        sqa.forward_v5(*_args(good_inputs()), 512, 3)


@pytest.mark.parametrize("mutation", ["value_shape", "page_size_arg", "meta_dtype", "batch_bt",
                                      "batch_sl", "empty"])
def test_launcher_contract_raises_runtime_error(fake_gpu, mutation):
    """reference csrc/small_q_attention_ext.cu:976-1002 (TORCH_CHECK -> RuntimeError)."""
    inp = good_inputs()
    page_size = 16
    if mutation == "value_shape":
        inp["value_cache"] = FakeTensor((11, 16, 8, 128))
    elif mutation == "page_size_arg":
        page_size = 8
    elif mutation == "meta_dtype":
        inp["seq_lens"] = FakeTensor((2,), dtype=torch.int64)
    elif mutation == "batch_bt":
        inp["block_tables"] = FakeTensor((3, 5), dtype=torch.int32)
    elif mutation == "batch_sl":
        inp["seq_lens"] = FakeTensor((1,), dtype=torch.int32)
    else:
        inp["key_cache"] = FakeTensor((0, 16, 8, 128))
        inp["value_cache"] = FakeTensor((0, 16, 8, 128))
    args = list(_args(inp))
    args[5] = page_size
    with pytest.raises(RuntimeError):
        sqa.forward_v0(*args)


def test_unsupported_page_size_and_row_count_raise_value_error(fake_gpu):
    with pytest.raises(ValueError):
        sqa.forward_v0(*_args(good_inputs(page=8))[:5], 8)
    with pytest.raises(ValueError):  # q_len 16 x group 8 = 128 rows > 64
        sqa.forward_v0(*_args(good_inputs(q_len=16, hq=32, hkv=4)))
