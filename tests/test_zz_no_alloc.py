"""vsk_sq8_search_noalloc (the no-allocation variant of vsk_sq8_search)
against vsk_sq8_search and against the oracle through the C ABI: scores and
ids bit for bit, on two calls in a row, the second with a smaller input;
through a context whose first device allocation is made to fail
(VSK_FAULT=alloc:1), which it must never reach; plus its error paths."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import Context, SQ8Database, VSKError
from vectorstorekit_amd._lib import check

pytestmark = pytest.mark.gpu


def _both(ctx, db, qc, k):
    """(scores, ids) of vsk_sq8_search and of vsk_sq8_search_noalloc on the
    same device query codes."""
    import torch

    nq = qc.shape[0]
    out = []
    for fn in (ctx.lib.vsk_sq8_search, ctx.lib.vsk_sq8_search_noalloc):
        s = torch.full((nq, k), 7, dtype=torch.int32, device="cuda")
        i = torch.full((nq, k), 7, dtype=torch.int64, device="cuda")
        torch.cuda.synchronize()
        check(ctx.handle, fn(ctx.handle, db.handle, qc.data_ptr(), nq, k, s.data_ptr(),
                             i.data_ptr()))
        out.append((s.cpu().numpy(), i.cpu().numpy()))
    return out


def test_noalloc_matches_sq8_search_twice(ctx):
    import torch

    rng = np.random.default_rng(11)
    # d = 100: padded to 128-byte rows, so the query codes are staged in
    # the static scratch too; 1,200 queries at k = 100 need three batches
    n, d = 200_000, 100
    codes = rng.integers(-128, 128, (n, d)).astype(np.int8)
    codes[9] = codes[4]  # a tie: the lower row id first
    db = SQ8Database(ctx, codes)
    q1 = torch.from_numpy(rng.integers(-128, 128, (1200, d)).astype(np.int8)).cuda()
    q1[0] = torch.from_numpy(codes[4]).cuda()
    print("noalloc call 1: n=200000 d=100 nq=1200 k=100", flush=True)
    (a_s, a_i), (b_s, b_i) = _both(ctx, db, q1, 100)
    np.testing.assert_array_equal(b_i, a_i)
    np.testing.assert_array_equal(b_s, a_s)
    assert a_i[0, 0] == 4 and a_i[0, 1] == 9
    os_, oi = O.sq8_search(q1.cpu().numpy(), codes, 100)
    np.testing.assert_array_equal(b_i, oi)
    np.testing.assert_array_equal(b_s, os_)
    # second call, smaller input: the array keeps the first call's contents
    q2 = q1[:37, :].contiguous()
    print("noalloc call 2: nq=37 k=10", flush=True)
    (a_s, a_i), (b_s, b_i) = _both(ctx, db, q2, 10)
    np.testing.assert_array_equal(b_i, a_i)
    np.testing.assert_array_equal(b_s, a_s)
    os_, oi = O.sq8_search(q2.cpu().numpy(), codes, 10)
    np.testing.assert_array_equal(b_i, oi)
    np.testing.assert_array_equal(b_s, os_)


def test_noalloc_allocates_nothing():
    """The database is made on one context; the no-allocation call runs on a
    second context whose first device allocation fails (VSK_FAULT=alloc:1):
    it succeeds, twice, and its results equal the oracle's, so it made no
    allocation.  vsk_sq8_search on that context does allocate (its scratch)
    and reports the injected outOfMemory."""
    import torch

    rng = np.random.default_rng(14)
    n, d = 300_000, 128
    codes = rng.integers(-128, 128, (n, d)).astype(np.int8)
    owner = Context(0)
    db = SQ8Database(owner, codes)
    old = os.environ.get("VSK_FAULT")
    os.environ["VSK_FAULT"] = "alloc:1"
    try:
        armed = Context(0)
    finally:
        if old is None:
            del os.environ["VSK_FAULT"]
        else:
            os.environ["VSK_FAULT"] = old
    for nq, k in ((700, 100), (20, 7)):
        q = torch.from_numpy(rng.integers(-128, 128, (nq, d)).astype(np.int8)).cuda()
        s = torch.full((nq, k), 7, dtype=torch.int32, device="cuda")
        i = torch.full((nq, k), 7, dtype=torch.int64, device="cuda")
        torch.cuda.synchronize()
        print(f"noalloc on an alloc-armed context: nq={nq} k={k}", flush=True)
        check(armed.handle, armed.lib.vsk_sq8_search_noalloc(
            armed.handle, db.handle, q.data_ptr(), nq, k, s.data_ptr(), i.data_ptr()))
        os_, oi = O.sq8_search(q.cpu().numpy(), codes, k)
        np.testing.assert_array_equal(i.cpu().numpy(), oi)
        np.testing.assert_array_equal(s.cpu().numpy(), os_)
    with pytest.raises(VSKError) as e:
        check(armed.handle, armed.lib.vsk_sq8_search(
            armed.handle, db.handle, q.data_ptr(), 20, 7, s.data_ptr(), i.data_ptr()))
    assert e.value.kind == "outOfMemory"
    armed.close()
    db.free()
    owner.close()


def test_noalloc_small_db_and_k_past_rows(ctx):
    import torch

    rng = np.random.default_rng(12)
    codes = rng.integers(-128, 128, (50, 64)).astype(np.int8)
    db = SQ8Database(ctx, codes)
    q = torch.from_numpy(rng.integers(-128, 128, (5, 64)).astype(np.int8)).cuda()
    print("noalloc small: n=50 d=64 nq=5 k=64", flush=True)
    (a_s, a_i), (b_s, b_i) = _both(ctx, db, q, 64)
    np.testing.assert_array_equal(b_i, a_i)
    np.testing.assert_array_equal(b_s, a_s)
    assert (b_i[:, 50:] == -1).all()


def test_noalloc_rejects_host_buffers(ctx):
    rng = np.random.default_rng(13)
    codes = rng.integers(-128, 128, (100, 32)).astype(np.int8)
    db = SQ8Database(ctx, codes)
    qc = rng.integers(-128, 128, (2, 32)).astype(np.int8)
    s = np.empty((2, 5), np.int32)
    i = np.empty((2, 5), np.int64)
    with pytest.raises(VSKError) as e:
        check(ctx.handle, ctx.lib.vsk_sq8_search_noalloc(ctx.handle, db.handle,
                                                         qc.ctypes.data, 2, 5,
                                                         s.ctypes.data, i.ctypes.data))
    assert e.value.status == -2


def test_noalloc_rejects_oversized_query(ctx):
    """A single query whose padded codes exceed the 64 MiB array (d is not a
    multiple of 32, so the query codes need a padded copy in the array)."""
    import torch

    d = (64 << 20) + 1
    codes = torch.zeros((1, d), dtype=torch.int8, device="cuda")
    db = SQ8Database(ctx, codes)
    q = torch.zeros((1, d), dtype=torch.int8, device="cuda")
    s = torch.empty((1, 1), dtype=torch.int32, device="cuda")
    i = torch.empty((1, 1), dtype=torch.int64, device="cuda")
    with pytest.raises(VSKError) as e:
        check(ctx.handle, ctx.lib.vsk_sq8_search_noalloc(ctx.handle, db.handle, q.data_ptr(),
                                                         1, 1, s.data_ptr(), i.data_ptr()))
    assert e.value.status == -9
