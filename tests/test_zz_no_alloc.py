"""The allocation-free rows product (sm_plate_product_rows_noalloc) against sm_plate_product_rows (GPU).

Both go through the C ABI on the same plate and rows; the second call of each pair has fewer rows than the
first, so the static scratch still holds the first call's larger light when the second runs.  Both must equal
the exact integer product (base2.py:29-32) of the same rows.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nin,nout", [(768, 2304), (3072, 768), (768, 50257)])
def test_noalloc_rows_product_matches_rows_product(sm, nin, nout):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(nin + nout)
    w = rng.integers(-32767, 32768, (nin, nout), dtype=np.int16)
    e = rng.integers(-16, -8, nout, dtype=np.int32)
    b = rng.integers(-(1 << 20), 1 << 20, nout, dtype=np.int64)
    plate = sm.Plate(w, e, b, tile_cols=0)
    try:
        for rows in (64, 5):
            x = rng.integers(-32768, 32769, (rows, nin), dtype=np.int64)
            x[0, :7] = 32768                         # the lights a byte pair cannot hold
            x[rows - 1, -5:] = -32768
            want = x @ w.astype(np.int64)           # exact: every partial sum is below 2^43
            dx = torch.from_numpy(x).cuda()
            ref = torch.zeros((rows, nout), dtype=torch.int64, device="cuda")
            got = torch.zeros((rows, nout), dtype=torch.int64, device="cuda")
            plate.product_rows(dx.data_ptr(), rows, ref.data_ptr())
            plate.product_rows_noalloc(dx.data_ptr(), rows, got.data_ptr())
            torch.cuda.synchronize()
            ref_h, got_h = ref.cpu().numpy(), got.cpu().numpy()
            assert np.array_equal(ref_h, want), f"rows product, {rows} rows"
            assert np.array_equal(got_h, ref_h), f"allocation-free rows product, {rows} rows"
    finally:
        plate.close()


def test_noalloc_rejects_more_rows_than_its_scratch(sm):
    rng = np.random.default_rng(3)
    w = rng.integers(-32767, 32768, (768, 768), dtype=np.int16)
    plate = sm.Plate(w, np.full(768, -12, np.int32), np.zeros(768, np.int64), tile_cols=0)
    try:
        with pytest.raises(sm.SmError, match="rows must be in"):
            plate.product_rows_noalloc(1, 65, 1)      # (never dereferenced: the row count is refused first)
    finally:
        plate.close()
