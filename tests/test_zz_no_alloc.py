"""vsk_sq8_search_noalloc (the no-allocation variant of vsk_sq8_search)
against vsk_sq8_search through the C ABI: scores and ids bit for bit, on two
calls in a row, the second with a smaller input, plus its error paths."""
import ctypes

import numpy as np
import pytest

from vectorstorekit_amd import SQ8Database, VSKError
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
    # second call, smaller input: the array keeps the first call's contents
    q2 = q1[:37, :].contiguous()
    print("noalloc call 2: nq=37 k=10", flush=True)
    (a_s, a_i), (b_s, b_i) = _both(ctx, db, q2, 10)
    np.testing.assert_array_equal(b_i, a_i)
    np.testing.assert_array_equal(b_s, a_s)


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
