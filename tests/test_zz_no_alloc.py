"""forge_layer_norm_bwd_noalloc: the LayerNorm backward that allocates
nothing (dgamma/dbeta partial rows in the library's static device scratch).

Called through the C ABI and compared bit for bit with forge_layer_norm_bwd
on the same inputs, on consecutive calls whose second input is smaller (the
scratch keeps the previous call's contents), over the register and the
looping paths, with dgamma/dbeta, with one of them and with none; a shape
whose partial rows exceed the scratch is refused with FORGE_EINVAL."""
import numpy as np
import pytest

import oxforge
from oxforge import synth
from oxforge._lib import call

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def _sl(a):
    return oxforge._sl(a)


def run(rt, entry, x, dy, gam, rows, cols, want_g=True, want_b=True):
    dX, dDY = rt.array(x), rt.array(dy)
    dgam = rt.array(gam) if gam is not None else None
    dDX = rt.array(np.full((rows, cols), np.nan, np.float32))
    pg = rt.array(np.full((cols,), np.nan, np.float32)) if want_g else None
    pb = rt.array(np.full((cols,), np.nan, np.float32)) if want_b else None
    call(entry, rt.handle, None, dX.slice, dDY.slice, _sl(dgam), dDX.slice, _sl(pg), _sl(pb),
         rows, cols, 1e-5)
    out = (dDX.numpy(), pg.numpy() if want_g else None, pb.numpy() if want_b else None)
    for d in (dX, dDY, dgam, dDX, pg, pb):
        if d is not None:
            d.recycle()
    return out


def same(a, b):
    for u, v in zip(a, b):
        if u is None:
            assert v is None
        else:
            assert np.array_equal(u, v)


# (rows, cols): the C2 shape, then a smaller one on the same scratch; the
# looping path (cols % 4 != 0, and 16-byte-unaligned widths); 2048 columns
# (eight float4 per lane); a single row.
SEQUENCES = [
    [(4096, 1024), (300, 1024)],
    [(2048, 2048), (64, 2048), (1, 2048)],
    [(513, 1001), (33, 1001)],
    [(257, 1024), (256, 7)],
]


@pytest.mark.parametrize("shapes", SEQUENCES)
def test_noalloc_matches_allocating_entry_on_consecutive_calls(rt, shapes):
    for k, (rows, cols) in enumerate(shapes):
        say(f"layer_norm_bwd_noalloc {rows}x{cols} (call {k + 1} of {len(shapes)})")
        x = synth.normal((rows, cols), 100 + k)
        dy = synth.normal((rows, cols), 200 + k)
        gam = synth.normal((cols,), 300 + k, 1.0, 0.1)
        for want_g, want_b in ((True, True), (True, False), (False, True), (False, False)):
            ref = run(rt, "forge_layer_norm_bwd", x, dy, gam, rows, cols, want_g, want_b)
            got = run(rt, "forge_layer_norm_bwd_noalloc", x, dy, gam, rows, cols, want_g, want_b)
            same(got, ref)
        ref = run(rt, "forge_layer_norm_bwd", x, dy, None, rows, cols)
        got = run(rt, "forge_layer_norm_bwd_noalloc", x, dy, None, rows, cols)
        same(got, ref)


def test_noalloc_refuses_shapes_beyond_the_scratch(rt):
    say("layer_norm_bwd_noalloc refuses 1024x4096")
    rows, cols = 1024, 4096  # looping path: 1024 partial rows x 4096 x 2 > 2^21 floats
    dX, dDY, dDX = rt.empty((rows, cols)), rt.empty((rows, cols)), rt.empty((rows, cols))
    pg, pb = rt.empty((cols,)), rt.empty((cols,))
    with pytest.raises(oxforge.ForgeError) as e:
        call("forge_layer_norm_bwd_noalloc", rt.handle, None, dX.slice, dDY.slice,
             oxforge._lib.NULL_SLICE, dDX.slice, pg.slice, pb.slice, rows, cols, 1e-5)
    assert e.value.status == 1 and "scratch" in str(e.value)
    # Without dgamma/dbeta there are no partial rows: the same shape runs.
    x = synth.normal((rows, cols), 7)
    dX.upload(x)
    dDY.upload(x)
    call("forge_layer_norm_bwd_noalloc", rt.handle, None, dX.slice, dDY.slice,
         oxforge._lib.NULL_SLICE, dDX.slice, oxforge._lib.NULL_SLICE, oxforge._lib.NULL_SLICE,
         rows, cols, 1e-5)
    ref = rt.empty((rows, cols))
    rt.layer_norm_bwd(dX, dDY, ref, rows, cols)
    assert np.array_equal(dDX.numpy(), ref.numpy())
