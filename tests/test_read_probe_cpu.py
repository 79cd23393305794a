"""The bench's streaming-read probe library (``libsqa_probe.so``, ``read_probe.hip``)
on the CPU: it loads, carries its source stamp, and rejects bad arguments before
any device call. ``libsqa.so`` (the product) no longer exports the probe."""

import ctypes

import pytest

import read_probe
from small_q_attention_amd import _lib


@pytest.fixture(scope="module")
def probe():
    return read_probe.load(build_if_missing=True)


def test_probe_library_is_stamped_with_its_sources(probe):
    assert read_probe.source_hash() in probe.sqa_probe_version().decode()


@pytest.mark.parametrize("args,msg", [
    ((0, 4096, 4096, 1), "null pointer"),
    ((4096, 4096, 0, 1), "null pointer"),
    ((4096, 4096, 4096, 0), "blocks"),
    ((4096, 4096, 4096, 65537), "blocks"),
    ((4104, 4096, 4096, 1), "aligned"),
    ((4096, 4096, 4098, 1), "aligned"),
    ((4096, 0, 4096, 1), "multiple"),
    ((4096, 4096 + 16, 4096, 2), "multiple"),
])
def test_read_probe_rejects_bad_arguments_without_a_gpu(probe, args, msg):
    data, nbytes, sink, blocks = args
    assert probe.sqa_read_probe(data, nbytes, sink, blocks, None) == 1
    assert msg in probe.sqa_probe_last_error().decode()


def test_product_library_does_not_export_the_probe():
    lib = ctypes.CDLL(str(_lib.load(build_if_missing=True)._name))
    assert not hasattr(lib, "sqa_read_probe")
