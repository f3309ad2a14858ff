"""Seeded random-shape sweeps of the GEMM and row kernels against the CPU
oracle, so that shape-dependent choices (tile, split-K, guarded fallback,
register or looping row path, masked lanes, unaligned views, partial-sum
grids) meet the same bars on shapes no list names.  Bars as in
test_gpu_kernels.py: GEMM max|C - C64| / max|C64| <= 1e-4 and componentwise
|C - C64| / (|A| |B|) <= 1e-4; row kernels 1e-5 absolute, column sums
1e-5 sqrt(rows)."""
import numpy as np
import pytest

import oxforge
from oxforge import synth
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL_ROW = 1e-5


def say(msg):
    print(f"[case] {msg}", flush=True)


def _dim(rng, hi):
    # Mostly multiples of 16/32/64 (the unguarded tiles), sometimes ragged.
    d = int(rng.integers(1, hi + 1))
    r = rng.random()
    if r < 0.3:
        d = max(64, d // 64 * 64)
    elif r < 0.5:
        d = max(32, d // 32 * 32)
    return d


def _view(rt, host, off):
    """host placed `off` floats into a fresh buffer (off > 0: not 16-byte
    aligned), and the view of it."""
    buf = rt.array(np.concatenate([np.zeros(off, np.float32), host.ravel()]))
    return buf, buf.view(off, host.shape)


@pytest.mark.parametrize("seed", range(6))
def test_gemm_random_shapes(rt, seed):
    rng = np.random.default_rng(1000 + seed)
    for case in range(25):
        M, N, K = _dim(rng, 700), _dim(rng, 700), _dim(rng, 2500)
        if rng.random() < 0.15:
            K = int(rng.integers(2048, 9000)) // 32 * 32  # split-K territory
            M, N = 64 * int(rng.integers(1, 3)), 64 * int(rng.integers(1, 3))
        ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
        off = int(rng.choice([0, 0, 0, 1, 3]))
        say(f"seed {seed} case {case}: {M}x{N}x{K} ta={ta} tb={tb} off={off}")
        A = synth.uniform((K, M) if ta else (M, K), seed * 100 + case)
        B = synth.uniform((N, K) if tb else (K, N), seed * 100 + case + 50)
        bufA, dA = _view(rt, A, off)
        dB = rt.array(B)
        bias = synth.uniform((N,), 7) if rng.random() < 0.5 else None
        res = synth.uniform((M, N), 8) if rng.random() < 0.5 else None
        act = int(rng.choice([oxforge.ACT_IDENTITY, oxforge.ACT_RELU]))
        dbias = rt.array(bias) if bias is not None else None
        dres = rt.array(res) if res is not None else None
        dC = rt.empty((M, N))
        rt.gemm_ex(dA, dB, dC, M, N, K, trans_a=bool(ta), trans_b=bool(tb), bias=dbias,
                   residual=dres, activation=act)
        ref = orc.gemm_f64(A, B, ta, tb)
        scale = np.abs(A.T if ta else A).astype(np.float64) @ np.abs(B.T if tb else B).astype(np.float64)
        if bias is not None:
            ref = ref + bias
            scale = scale + np.abs(bias)
        if res is not None:
            ref = ref + res
            scale = scale + np.abs(res)
        if act == oxforge.ACT_RELU:
            ref = np.maximum(ref, 0.0)
        C = dC.numpy().astype(np.float64)
        err = np.abs(C - ref)
        rel_max = float(err.max() / max(np.abs(ref).max(), 1e-30))
        comp = float((err / np.maximum(scale, 1e-30)).max())
        assert rel_max <= 1e-4 and comp <= 1e-4, (M, N, K, ta, tb, off, rel_max, comp)
        for d in (bufA, dB, dC) + tuple(x for x in (dbias, dres) if x is not None):
            d.recycle()


@pytest.mark.parametrize("seed", range(6))
def test_row_kernels_random_shapes(rt, seed):
    rng = np.random.default_rng(2000 + seed)
    for case in range(20):
        rows = int(rng.integers(1, 400))
        cols = int(rng.choice([int(rng.integers(1, 5000)), 4 * int(rng.integers(1, 1024))]))
        off = int(rng.choice([0, 0, 1, 2]))
        affine = bool(rng.random() < 0.6)
        say(f"seed {seed} case {case}: {rows}x{cols} off={off} affine={affine}")
        x = synth.normal((rows, cols), seed * 100 + case)
        dy = synth.normal((rows, cols), seed * 100 + case + 50)
        gam = synth.normal((cols,), 3, 1.0, 0.1) if affine else None
        bet = synth.normal((cols,), 4, 0.0, 0.1) if affine else None
        dgam = rt.array(gam) if affine else None
        dbet = rt.array(bet) if affine else None
        bufs = []

        def view(h):
            b, v = _view(rt, h, off)
            bufs.append(b)
            return v

        v = view(x)
        rt.softmax_rows(v, rows, cols)
        p = v.numpy()
        assert np.max(np.abs(p - orc.softmax_rows(x))) <= TOL_ROW
        dd = view(np.zeros_like(x))
        rt.softmax_rows_bwd(view(p), view(dy), dd, rows, cols)
        assert np.max(np.abs(dd.numpy() - orc.softmax_rows_backward(p, dy))) <= TOL_ROW

        v = view(x)
        rt.layer_norm(v, rows, cols, dgam, dbet)
        assert np.max(np.abs(v.numpy() - orc.layer_norm(x, gam, bet))) <= TOL_ROW
        v = view(x)
        rt.rms_norm(v, rows, cols, dgam)
        assert np.max(np.abs(v.numpy() - orc.rms_norm(x, gam))) <= TOL_ROW

        col_tol = TOL_ROW * max(1.0, np.sqrt(rows))
        dx = view(np.zeros_like(x))
        pg, pb = rt.empty((cols,)), rt.empty((cols,))
        rt.layer_norm_bwd(view(x), view(dy), dx, rows, cols, gamma=dgam, dgamma=pg, dbeta=pb)
        rdx, rdg, rdb = orc.layer_norm_backward(x, dy, gam, want_params=True)
        assert np.max(np.abs(dx.numpy() - rdx)) <= TOL_ROW
        assert np.max(np.abs(pg.numpy() - rdg)) <= col_tol
        assert np.max(np.abs(pb.numpy() - rdb)) <= col_tol
        rt.rms_norm_bwd(view(x), view(dy), dx, rows, cols, gamma=dgam, dgamma=pg)
        rdx, rdg = orc.rms_norm_backward(x, dy, gam, want_params=True)
        assert np.max(np.abs(dx.numpy() - rdx)) <= TOL_ROW
        assert np.max(np.abs(pg.numpy() - rdg)) <= col_tol
        for d in bufs + [pg, pb] + [d for d in (dgam, dbet) if d is not None]:
            d.recycle()
