"""CPU properties of the balanced plan's layout as ``tests/test_gpu_plans.py`` states
it (the model the device's (first slot, count) table is checked against), with and
without seam gaps: every sequence's pages map to one run of consecutive slots, no
two sequences share a slot, every slot is below num_splits, uniform batches are
laid out exactly as without gaps, and an item that spans a gapped sequence start
holds ``seam`` fewer pages than a full item."""

import random

from tests.test_gpu_plans import SEAM_PAGES, _packed_layout


def test_slots_are_disjoint_runs_below_num_splits():
    rng = random.Random(7)
    for _ in range(400):
        batch = rng.randint(2, 60)
        lens = [rng.choice([0, rng.randint(1, 700), rng.randint(1, 40000)]) for _ in range(batch)]
        max_pages = max((n + 15) // 16 for n in lens)
        items = max(rng.choice([1, 2, 3, 7, 64, 128]), -(-batch * max_pages // 2048))
        for seam in (0, SEAM_PAGES, 9):
            P, slots = _packed_layout(lens, items, seam=seam)
            used = []
            for b, s in enumerate(slots):
                if s:
                    assert s == list(range(s[0], s[0] + len(s))), (lens, b)
                used += s
            assert len(used) == len(set(used))
            assert not used or max(used) < items + batch
            assert 4 <= P <= 2048


def test_uniform_batches_get_no_gaps():
    for n, batch, items in [(333, 9, 5), (8192, 4, 128), (32768, 16, 128), (1000, 3, 128)]:
        assert _packed_layout([n] * batch, items, seam=SEAM_PAGES) == \
            _packed_layout([n] * batch, items, seam=0)


def test_a_gap_takes_its_pages_from_the_item_that_spans_the_start():
    # Two sequences whose boundary falls inside an item: with the gap, that
    # item's pages in the two sequences add up to P - seam; without, to P.
    lens = [16 * 1000, 16 * 1100]
    for seam in (0, SEAM_PAGES):
        P, slots = _packed_layout(lens, 16, seam=seam)
        pages = [1000, 1100]
        start1 = 1000 + seam if 1000 % _packed_layout(lens, 16, seam=0)[0] else 1000
        item = slots[0][-1]  # the last item of sequence 0 (slot = item + 0)
        in0 = sum(1 for j in range(pages[0]) if j // P == item)
        in1 = sum(1 for j in range(pages[1]) if (start1 + j) // P == item)
        assert in0 + in1 == P - seam, (seam, P, in0, in1)
