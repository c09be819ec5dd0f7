"""Failure handling, forced from the host (VSK_FAULT=<kind>:<n>): the n-th
device allocation, launch check or end-of-call synchronisation of a context
reports an error although the GPU work itself ran normally.  Each injected
fault must surface as the status the reference's error vocabulary maps it
to (outOfMemory / executionFailed), and the same context must then answer
a search exactly as the oracle does (recovery: the fault fires once, the
call's partial state is dropped)."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import Context, VectorDatabase, VSKError

OUT_OF_MEMORY, EXECUTION_FAILED = -5, -6  # vsk_status (vsk_hip.h)

pytestmark = pytest.mark.gpu


def _armed(spec):
    old = os.environ.get("VSK_FAULT")
    os.environ["VSK_FAULT"] = spec
    try:
        return Context(0)
    finally:
        if old is None:
            del os.environ["VSK_FAULT"]
        else:
            os.environ["VSK_FAULT"] = old


@pytest.mark.parametrize("spec,status", [("alloc:1", OUT_OF_MEMORY),
                                         ("alloc:3", OUT_OF_MEMORY),
                                         ("launch:1", EXECUTION_FAILED),
                                         ("launch:4", EXECUTION_FAILED),
                                         ("sync:1", EXECUTION_FAILED),
                                         ("sync:2", EXECUTION_FAILED)])
def test_injected_fault_maps_and_recovers(spec, status):
    rng = np.random.default_rng(21)
    x = rng.standard_normal((3000, 40)).astype(np.float32)
    q = rng.standard_normal((25, 40)).astype(np.float32)
    ctx = _armed(spec)
    raised = None
    try:
        for _ in range(3):  # enough events for every spec above
            db = VectorDatabase(ctx, x)
            db.search(q, 10, "euclideanSquared")
            db.free()
    except VSKError as e:
        raised = e
    assert raised is not None, "the armed fault did not fire"
    assert raised.status == status, raised
    assert "injected fault" in str(raised)
    # the context recovers: a full upload and search match the oracle
    db = VectorDatabase(ctx, x)
    gd, gi = db.search(q, 10, "euclideanSquared")
    od, oi = O.search_flat(q, x, 10, O.L2SQ)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    db.free()
    ctx.close()


def test_unarmed_and_malformed_specs_do_nothing():
    rng = np.random.default_rng(22)
    x = rng.standard_normal((500, 8)).astype(np.float32)
    for spec in ("", "launch", "launch:0", "nothing:3", "sync:-2"):
        ctx = _armed(spec)
        db = VectorDatabase(ctx, x)
        gd, gi = db.search(x[:5], 3, "euclideanSquared")
        od, oi = O.search_flat(x[:5], x, 3, O.L2SQ)
        np.testing.assert_array_equal(gi, oi)
        db.free()
        ctx.close()


@pytest.mark.parametrize("spec", ["launch:3", "sync:2"])
def test_profile_reset_after_failed_profiled_call(spec):
    """With per-kernel timing on, a call that fails after some of its
    timers closed leaves no pending timings behind: vsk_profile_reset and
    the next call see clean statistics (the next call's timings name only
    statistics that exist)."""
    rng = np.random.default_rng(23)
    x = rng.standard_normal((4000, 32)).astype(np.float32)
    q = rng.standard_normal((30, 32)).astype(np.float32)
    ctx = _armed(spec)
    ctx.profile(True)
    db = VectorDatabase(ctx, x)
    raised = None
    try:
        for _ in range(3):
            db.search(q, 10, "euclideanSquared")
    except VSKError as e:
        raised = e
    assert raised is not None, "the armed fault did not fire"
    ctx.profile_reset()
    gd, gi = db.search(q, 10, "euclideanSquared")
    od, oi = O.search_flat(q, x, 10, O.L2SQ)
    np.testing.assert_array_equal(gi, oi)
    stats = ctx.profile_stats()
    assert stats and all(v[0] >= 1 for v in stats.values())
    db.free()
    ctx.close()
