"""CPU oracle for paged small-q (MTP) attention.

TEST INFRASTRUCTURE ONLY. Nothing in the product package
(``small_q_attention_amd``) imports this package. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
it, and only as the checker or as the timed CPU baseline, never as a fallback
for the HIP path.

Three independent restatements of
``/root/reference/src/small_q_attention/reference.py:10-74``:

* :func:`paged_mtp_attention_reference` (``oracle/reference.py``): loop-faithful
  torch restatement, same name, signature and ``ValueError`` conditions.
* :func:`attention_numpy` (``oracle/vectorized.py``): vectorized numpy version
  (float32 or float64), used at sizes the loop version is too slow for.
* :func:`attention_c64` (``oracle/cbrute.py`` over ``oracle/sqa_oracle.c``):
  scalar C brute force in double precision with OpenMP.

How each is pinned (all checks live in ``tests/test_oracle_*.py``):
known answers restated from the reference's own tests
(``tests/test_reference.py:9-45``, ``tests/test_reference_edges.py:17-78``,
the zero fixture corrected), closed forms (uniform softmax gives the mean of
the visible V rows, ``seq_len == q_len`` gives ``V[0]`` for row 0, one visible
key gives that key's V), invariants (page-table permutation, GQA head
symmetry) and agreement of the three restatements with each other on
seeded inputs. The fp16-CPU-input path of the reference (``reference.py:68-70``:
fp16 logits, probabilities cast back to fp16, fp16 PV) is pinned by closed
forms in ``tests/test_checker_pinned.py``: a uniform softmax over 4 and 8 keys,
3:1 weights and a dominant key, where every weight and product is exact in
fp16, give the fp32 path's result rounded to fp16 bit for bit.
"""

from .reference import paged_mtp_attention_reference
from .vectorized import attention_numpy, gather_sequence
from .cbrute import attention_c64, c_oracle_available

__all__ = [
    "paged_mtp_attention_reference",
    "attention_numpy",
    "gather_sequence",
    "attention_c64",
    "c_oracle_available",
]
