"""The allocation-free selection entry point, w4h_op_select_noalloc, against w4h_op_select.

Both run the same partial and merge kernels with the same number of partials per row, so the records
must be bit-identical.  Two calls in a row, the second with fewer and shorter rows than the first, show
that what the first left in the library's fixed partials array does not leak into the second.  A
request beyond the array's row limit is refused with W4H_ERR_INVALID.
"""

import ctypes

import numpy as np
import pytest

from whisper4j_amd import _lib

pytestmark = pytest.mark.gpu
FIELDS = ("argmax", "max_logit", "logsumexp", "probe_logit", "raw_logsumexp")


def _case(rows, n, seed):
    rng = np.random.default_rng(seed)
    lg = rng.standard_normal((rows, n)).astype(np.float32)
    lg[:, n // 3] = lg.max(axis=1) + 1.0  # a tie for the maximum: the lower index must win
    lg[:, 2 * n // 3] = lg[:, n // 3]
    mw = (n + 31) // 32
    mask = np.zeros((rows, mw), np.uint32)
    for r in range(rows):
        for t in rng.integers(0, n, 40):
            mask[r, t >> 5] |= np.uint32(1 << (int(t) & 31))
    mask[0, (n // 3) >> 5] |= np.uint32(1 << ((n // 3) & 31))  # row 0: the first maximum masked
    return lg, mask


def _host(gpu, lg, mask, k):
    rows, n = lg.shape
    out = (_lib.StepOut * rows)()
    _lib.check(gpu.lib().w4h_op_select(lg.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), rows, n,
                                       mask.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), k, out))
    return list(out)


def _noalloc(gpu, lg, mask, k):
    from whisper4j_amd.device import DeviceArray

    rows, n = lg.shape
    nbytes = ctypes.sizeof(_lib.StepOut) * rows
    with DeviceArray(lg) as dl, DeviceArray(mask) as dm, DeviceArray(np.zeros(nbytes, np.uint8)) as do:
        _lib.check(gpu.lib().w4h_op_select_noalloc(dl.address, rows, n, dm.address, k, do.address, None))
        raw = do.numpy()  # a default-stream copy: ordered after the selection
    return list((_lib.StepOut * rows).from_buffer_copy(raw.tobytes()))


def _same(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        for f in FIELDS:
            assert getattr(x, f) == getattr(y, f), f
        assert list(x.topk_ids) == list(y.topk_ids)
        assert list(x.topk_logits) == list(y.topk_logits)


def test_select_noalloc_matches_select(gpu):
    for rows, n, k, seed in ((20, 51866, 8, 1), (7, 1000, 3, 2)):
        lg, mask = _case(rows, n, seed)
        want = _host(gpu, lg, mask, k)
        got = _noalloc(gpu, lg, mask, k)
        _same(got, want)
        assert got[1].argmax == n // 3  # the tie keeps the lower index
        assert got[0].argmax == 2 * n // 3  # its twin when the first is masked
        print(f"[no-alloc] rows {rows} n {n} k {k}: records bit-identical to w4h_op_select", flush=True)


def test_select_noalloc_rejects_too_many_rows(gpu):
    n = 64
    rc = gpu.lib().w4h_op_select_noalloc(ctypes.c_void_p(16), _lib.W4H_SELECT_MAX_ROWS + 1, n, None, 1,
                                         ctypes.c_void_p(16), None)
    assert rc == _lib.W4H_ERR_INVALID
    assert b"scratch" in gpu.lib().w4h_last_error()
