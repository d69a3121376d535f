"""ih_argmax_rows_noalloc (no allocation, a static per-device scratch) against ih_argmax_rows.

No counterpart in the reference: the entry point exists for callers that cannot allocate device memory. Two calls in a
row, the second with fewer rows (the scratch keeps the first call's partials: nothing may leak into the second), plus
the size limit.
"""
import numpy as np
import pytest

from ingot_amd._lib import IH_EINVAL, IngotError, check, lib

pytestmark = pytest.mark.gpu

MAX_ROWS = 256


def run(ctx, fn, x):
    rows, N = x.shape
    dx = ctx.to_device(np.ascontiguousarray(x, np.float32))
    out = ctx.buffer(rows * 4).fill(0xFF)
    check(fn(ctx.handle, dx.ptr, rows, N, out.ptr))
    r = out.download(np.uint32, (rows,))
    dx.free()
    out.free()
    return r


def test_noalloc_argmax_matches_allocating_entry_point(ctx):
    g = np.random.default_rng(42)
    big = g.normal(0, 1, size=(MAX_ROWS, 32000)).astype(np.float32)
    big[3, 100] = big[3, 20000] = 99.0  # a tie across chunks
    big[7, :] = -np.inf
    small = g.normal(0, 1, size=(17, 151936)).astype(np.float32)
    small[0, :] = np.nan
    small[0, 5] = 1.0
    for x in (big, small):
        want = run(ctx, lib().ih_argmax_rows, x)
        got = run(ctx, lib().ih_argmax_rows_noalloc, x)
        assert np.array_equal(got, want)
        finite = ~np.any(np.isnan(x), axis=1)  # numpy's argmax returns the first NaN; the rule here never picks one
        assert np.array_equal(want[finite], np.argmax(x[finite], axis=1).astype(np.uint32))
    assert run(ctx, lib().ih_argmax_rows_noalloc, small)[0] == 5


def test_noalloc_argmax_rejects_rows_beyond_the_scratch(ctx):
    x = ctx.buffer((MAX_ROWS + 1) * 8 * 4)
    out = ctx.buffer((MAX_ROWS + 1) * 4)
    with pytest.raises(IngotError) as e:
        check(lib().ih_argmax_rows_noalloc(ctx.handle, x.ptr, MAX_ROWS + 1, 8, out.ptr))
    assert e.value.code == IH_EINVAL
    x.free()
    out.free()
