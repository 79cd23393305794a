"""MI355X-native paged small-q (speculative-decoding "MTP") attention.

The op boundary mirrors ``small_q_attention.cuda`` of the reference
(``/root/reference/src/small_q_attention/cuda.py``): ``load_v0..load_v5`` and
``forward_v0..forward_v5``, plus :func:`paged_mtp_attention`, the native entry
with the automatic split plan. All of them run the gfx950 kernels of
``libsqa.so`` through the ``sqa::paged_mtp_attention`` torch custom op.

The CPU oracle (the reference's ``paged_mtp_attention_reference``) is test
infrastructure and lives in the top-level ``oracle`` package; this package
never imports it.
"""

from .cuda import (  # noqa: F401
    forward_v0,
    forward_v1,
    forward_v2,
    forward_v3,
    forward_v4,
    forward_v5,
    load_v0,
    load_v1,
    load_v2,
    load_v3,
    load_v4,
    load_v5,
    paged_mtp_attention,
)

__version__ = "0.1.0"
