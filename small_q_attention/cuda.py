"""``small_q_attention.cuda``: the reference's op module path over this build.

Re-exports ``load_v0..load_v5`` and ``forward_v0..forward_v5`` (the names of
``/root/reference/src/small_q_attention/cuda.py``) from
:mod:`small_q_attention_amd.cuda`; they are the same function objects, with the
reference's parameter order, defaults and exceptions.
"""

from small_q_attention_amd.cuda import (  # noqa: F401
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

__all__ = [
    "load_v0", "load_v1", "load_v2", "load_v3", "load_v4", "load_v5",
    "forward_v0", "forward_v1", "forward_v2", "forward_v3", "forward_v4", "forward_v5",
    "paged_mtp_attention",
]
