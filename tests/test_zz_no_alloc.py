"""forge_layer_norm_bwd_noalloc: the LayerNorm backward that allocates
nothing (dgamma/dbeta partial rows in the library's static device scratch).

Called through the C ABI and compared bit for bit with forge_layer_norm_bwd
on the same inputs, on consecutive calls whose second input is smaller (the
scratch keeps the previous call's contents), over the register and the
looping paths, with dgamma/dbeta, with one of them and with none; a shape
whose partial rows exceed the scratch is refused with FORGE_EINVAL."""
import ctypes

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


def unaligned(rt, host):
    """A device copy of host starting one float past a 16-byte boundary."""
    base = rt.empty((host.size + 1,))
    view = base.view(1, host.shape)
    view.upload(np.ascontiguousarray(host, np.float32))
    return base, view


def run(rt, entry, x, dy, gam, rows, cols, want_g=True, want_b=True, stream=None,
        misalign=False):
    if misalign:
        (bx, dX), (bdy, dDY) = unaligned(rt, x), unaligned(rt, dy)
    else:
        bx, bdy = None, None
        dX, dDY = rt.array(x), rt.array(dy)
    dgam = rt.array(gam) if gam is not None else None
    dDX = rt.array(np.full((rows, cols), np.nan, np.float32))
    pg = rt.array(np.full((cols,), np.nan, np.float32)) if want_g else None
    pb = rt.array(np.full((cols,), np.nan, np.float32)) if want_b else None
    call(entry, rt.handle, stream, dX.slice, dDY.slice, _sl(dgam), dDX.slice, _sl(pg), _sl(pb),
         rows, cols, 1e-5)
    rt.sync(stream)
    out = (dDX.numpy(), pg.numpy() if want_g else None, pb.numpy() if want_b else None)
    for d in ((bx, bdy) if misalign else (dX, dDY)) + (dgam, dDX, pg, pb):
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
# looping path (cols % 4 != 0, and 16-byte-unaligned widths), up to the
# widest shape it must take (1024 partial rows of 1001 columns); 2048 columns
# (eight float4 per lane); a single row.  The last flag puts x and dy one
# float past a 16-byte boundary, which sends 1024 columns down the looping
# path at its full 1024 partial rows.
SEQUENCES = [
    ([(4096, 1024), (300, 1024)], False),
    ([(2048, 2048), (64, 2048), (1, 2048)], False),
    ([(513, 1001), (33, 1001)], False),
    ([(4096, 1001), (1020, 1001)], False),
    ([(2048, 1024), (4096, 1024), (5, 1024)], True),
    ([(257, 1024), (256, 7)], False),
]


@pytest.mark.parametrize("shapes,misalign", SEQUENCES)
def test_noalloc_matches_allocating_entry_on_consecutive_calls(rt, shapes, misalign):
    for k, (rows, cols) in enumerate(shapes):
        say(f"layer_norm_bwd_noalloc {rows}x{cols}{' unaligned' if misalign else ''} "
            f"(call {k + 1} of {len(shapes)})")
        x = synth.normal((rows, cols), 100 + k)
        dy = synth.normal((rows, cols), 200 + k)
        gam = synth.normal((cols,), 300 + k, 1.0, 0.1)
        for want_g, want_b in ((True, True), (True, False), (False, True), (False, False)):
            ref = run(rt, "forge_layer_norm_bwd", x, dy, gam, rows, cols, want_g, want_b,
                      misalign=misalign)
            got = run(rt, "forge_layer_norm_bwd_noalloc", x, dy, gam, rows, cols, want_g, want_b,
                      misalign=misalign)
            same(got, ref)
        ref = run(rt, "forge_layer_norm_bwd", x, dy, None, rows, cols, misalign=misalign)
        got = run(rt, "forge_layer_norm_bwd_noalloc", x, dy, None, rows, cols, misalign=misalign)
        same(got, ref)


def workspace_floats(rt, stream):
    n = ctypes.c_size_t(12345)
    call("forge_stream_workspace_floats", rt.handle, stream, ctypes.byref(n))
    return n.value


def test_noalloc_leaves_a_fresh_stream_without_workspace(rt):
    """On a stream that has run nothing, the no-allocation entry point leaves
    the stream's workspace unallocated (the allocating entry point, run after
    it on the same stream, grows it: the check sees allocations), and its
    results still equal the allocating entry point's."""
    (s,) = rt.streams_create(1)
    rows, cols = 4096, 1024
    say(f"layer_norm_bwd_noalloc {rows}x{cols} on a fresh stream")
    x, dy = synth.normal((rows, cols), 61), synth.normal((rows, cols), 62)
    gam = synth.normal((cols,), 63, 1.0, 0.1)
    assert workspace_floats(rt, s) == 0
    got = run(rt, "forge_layer_norm_bwd_noalloc", x, dy, gam, rows, cols, stream=s)
    assert workspace_floats(rt, s) == 0
    ref = run(rt, "forge_layer_norm_bwd", x, dy, gam, rows, cols, stream=s)
    assert workspace_floats(rt, s) > 0
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
