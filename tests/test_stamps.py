"""The in-kernel timeline's reduction (ferrolm_amd.stamps.timeline), on
synthetic stamps: no GPU. Importing the module leaves the binding's library
choice alone."""
import os

import numpy as np


def test_import_leaves_the_library_choice_alone():
    before = os.environ.get("FERRO_STAMPS")
    import ferrolm_amd.stamps  # noqa: F401
    assert os.environ.get("FERRO_STAMPS") == before


def test_timeline_orders_launches_and_measures_spans():
    from ferrolm_amd.stamps import timeline
    ticks = np.zeros((4, 1024, 2), np.uint64)
    # slot 0: two workgroups, [100, 150] and [104, 170]; slot 1: unused;
    # slot 2 (launched first): three workgroups; slot 3: no record
    ticks[0, 0] = (100, 150)
    ticks[0, 1] = (104, 170)
    ticks[2, 0] = (10, 40)
    ticks[2, 1] = (12, 30)
    ticks[2, 2] = (11, 50)
    labels = ["gemv a", "attention", "gemv b", "merge"]
    rows = timeline(ticks, labels)
    assert [r[0] for r in rows] == ["gemv b", "gemv a"]  # by first entry; empty slots dropped
    lab, wgs, first, last, med = rows[0]
    assert (wgs, first, last) == (3, 10, 50)
    assert med == np.median([30, 18, 39])  # each workgroup's exit - entry
    assert rows[1][1:4] == (2, 100, 170) and rows[1][4] == np.median([50, 66])
