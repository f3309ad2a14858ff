"""Seeded random-shape sweeps of the GEMM and row kernels against the CPU
oracle, so that shape-dependent choices (tile, split-K, guarded fallback,
register or looping row path, masked lanes, unaligned views, partial-sum
grids) meet the same bars on shapes no list names.  Bars as in
test_gpu_kernels.py: GEMM max|C - C64| / max|C64| <= 1e-4 and componentwise
|C - C64| / (|A| |B|) <= 1e-4; row kernels 1e-5 absolute; the norm
backward's dgamma / dbeta (column sums over the rows) the larger of 1e-5
and twice the rounding bound of the kernels' summation tree
(rowbounds.layer_norm_param_bounds).  The LayerNorm forward and the LayerNorm / RMSNorm
backward dx are held to the larger of 1e-5 and twice the rounding bound of
their f32 formula (rowbounds.py): on rows whose values nearly coincide, r =
1/sqrt(var + eps) amplifies the f32 rounding of the mean past 1e-5 in any
f32 evaluation, the reference's included; for X ~ N(0,1) at 1024 columns
the bound is below 1e-5 and the bar is unchanged."""
import numpy as np
import pytest

import oxforge
import rowbounds as rb
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


def within(got, ref, bound):
    """|got - ref| <= max(1e-5, 2 * bound) everywhere; prints the worst
    element when it is not."""
    err = np.abs(np.asarray(got, np.float64) - ref)
    tol = rb.tolerance(bound, TOL_ROW)
    if np.all(err <= tol):
        return True
    i = np.unravel_index(np.argmax(err / tol), err.shape)
    print(f"  worst element {i}: error {err[i]:.3g}, tolerance {tol[i]:.3g}", flush=True)
    return False


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


@pytest.mark.parametrize("seed", range(4))
def test_gemm_sum_random_shapes(rt, seed):
    """forge_gemm_sum_f32 over random shapes, layouts, counts (2 or 3) and
    epilogues (bias, residual, ReLU): bit for bit forge_gemm_ex_f32 on the
    operands concatenated along K, whichever path the shape takes (the
    K-segment launch for tile-aligned shapes, the concatenating one for the
    rest and for K splits)."""
    rng = np.random.default_rng(5000 + seed)
    for case in range(12):
        aligned = rng.random() < 0.5
        if aligned:
            M, N = 64 * int(rng.integers(1, 9)), 64 * int(rng.integers(1, 9))
            K = 32 * int(rng.integers(1, 40))
        else:
            M, N, K = _dim(rng, 300), _dim(rng, 300), _dim(rng, 400)
        count = int(rng.integers(2, 4))
        ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
        say(f"seed {seed} case {case}: sum of {count} {M}x{N}x{K} ta={ta} tb={tb}")
        As = [synth.uniform((K, M) if ta else (M, K), seed * 100 + case * 7 + z)
              for z in range(count)]
        Bs = [synth.uniform((N, K) if tb else (K, N), seed * 100 + case * 7 + 50 + z)
              for z in range(count)]
        Ac = np.ascontiguousarray(np.concatenate(As, axis=0 if ta else 1))
        Bc = np.ascontiguousarray(np.concatenate(Bs, axis=1 if tb else 0))
        ep = {}
        if rng.random() < 0.5:
            ep["bias"] = rt.array(synth.uniform((N,), 7))
        if rng.random() < 0.5:
            ep["residual"] = rt.array(synth.uniform((M, N), 8))
        ep["activation"] = int(rng.choice([oxforge.ACT_IDENTITY, oxforge.ACT_RELU]))
        dC1, dC2 = rt.empty((M, N)), rt.empty((M, N))
        rt.gemm_sum([rt.array(a) for a in As], [rt.array(b) for b in Bs], dC1, M, N, K,
                    trans_a=bool(ta), trans_b=bool(tb), **ep)
        rt.gemm_ex(rt.array(Ac), rt.array(Bc), dC2, M, N, count * K, trans_a=bool(ta),
                   trans_b=bool(tb), **ep)
        assert np.array_equal(dC1.numpy(), dC2.numpy()), (M, N, K, count, ta, tb)


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
        assert within(v.numpy(), orc.layer_norm(x, gam, bet),
                      rb.layer_norm_forward_bound(x, gam, bet))
        v = view(x)
        rt.rms_norm(v, rows, cols, dgam)
        assert np.max(np.abs(v.numpy() - orc.rms_norm(x, gam))) <= TOL_ROW

        # dgamma / dbeta: the derived column-sum tolerance for this path
        # (x, dy views off a 16-byte boundary take the looping path).
        cu = rt.props()["cu_count"]
        bg, bb = rb.layer_norm_param_bounds(x, dy, cu, aligned=(off == 0))
        tg, tb = rb.tolerance(bg), rb.tolerance(bb)
        tr = rb.tolerance(rb.rms_norm_param_bound(x, dy, cu, aligned=(off == 0)))
        dx = view(np.zeros_like(x))
        pg, pb = rt.empty((cols,)), rt.empty((cols,))
        rt.layer_norm_bwd(view(x), view(dy), dx, rows, cols, gamma=dgam, dgamma=pg, dbeta=pb)
        rdx, rdg, rdb = orc.layer_norm_backward(x, dy, gam, want_params=True)
        assert within(dx.numpy(), rdx, rb.layer_norm_backward_bound(x, dy, gam))
        assert np.all(np.abs(pg.numpy() - rdg) <= tg)
        assert np.all(np.abs(pb.numpy() - rdb) <= tb)
        rt.rms_norm_bwd(view(x), view(dy), dx, rows, cols, gamma=dgam, dgamma=pg)
        rdx, rdg = orc.rms_norm_backward(x, dy, gam, want_params=True)
        assert within(dx.numpy(), rdx, rb.rms_norm_backward_bound(x, dy, gam))
        assert np.all(np.abs(pg.numpy() - rdg) <= tr)
        for d in bufs + [pg, pb] + [d for d in (dgam, dbet) if d is not None]:
            d.recycle()


@pytest.mark.parametrize("cols", [1, 2, 3, 5, 8, 33, 64, 256, 1024, 3000])
def test_row_norms_ill_conditioned(rt, cols):
    """Rows whose values nearly or exactly coincide, with means up to 30
    (r up to 1/sqrt(eps)), on the register path (aligned, cols % 4 == 0) and
    the looping path (a view one float off): the norms against the oracle
    within the rounding bounds of their f32 formulas (the column sums are
    left to the other tests: on such rows they inherit the same
    amplification)."""
    rng = np.random.default_rng(500 + cols)
    rows = 64
    for spread in (1e-2, 1e-4, 0.0):
        for off in (0, 1):
            affine = off == 0
            say(f"ill-conditioned {rows}x{cols} spread={spread} off={off} affine={affine}")
            m = rng.normal(0, 1, (rows, 1)) * rng.choice([1, 3, 10, 30], (rows, 1))
            x = (m + spread * rng.normal(0, 1, (rows, cols))).astype(np.float32)
            dy = rng.normal(0, 1, (rows, cols)).astype(np.float32)
            gam = (1 + 0.1 * rng.normal(0, 1, cols)).astype(np.float32) if affine else None
            bet = (0.1 * rng.normal(0, 1, cols)).astype(np.float32) if affine else None
            dgam = rt.array(gam) if affine else None
            dbet = rt.array(bet) if affine else None
            bufs = []

            def view(h):
                b, v = _view(rt, h, off)
                bufs.append(b)
                return v

            v = view(x)
            rt.layer_norm(v, rows, cols, dgam, dbet)
            assert within(v.numpy(), orc.layer_norm(x, gam, bet),
                          rb.layer_norm_forward_bound(x, gam, bet))
            v = view(x)
            rt.rms_norm(v, rows, cols, dgam)
            assert np.max(np.abs(v.numpy() - orc.rms_norm(x, gam))) <= TOL_ROW
            dx = view(np.zeros_like(x))
            rt.layer_norm_bwd(view(x), view(dy), dx, rows, cols, gamma=dgam)
            assert within(dx.numpy(), orc.layer_norm_backward(x, dy, gam),
                          rb.layer_norm_backward_bound(x, dy, gam))
            rt.rms_norm_bwd(view(x), view(dy), dx, rows, cols, gamma=dgam)
            assert within(dx.numpy(), orc.rms_norm_backward(x, dy, gam),
                          rb.rms_norm_backward_bound(x, dy, gam))
            for d in bufs + [d for d in (dgam, dbet) if d is not None]:
                d.recycle()


@pytest.mark.parametrize("seed", range(4))
def test_transformer_random_configs(rt, seed):
    """Random single-block configurations: sequence, hidden, FFN and output
    sizes (ragged ones take the guarded GEMM), LayerNorm or RMSNorm with or
    without gamma / beta, biases or none, each FFN activation, encoder or
    decoder inference (with or without forked Q/K/V streams) or the
    training step, and a score budget that forces query-chunked attention
    about half the time; output, input gradient and every parameter
    gradient against the f64 oracle at 1e-4 of the largest value, and the
    SGD identity on every updated parameter."""
    from oracle import executors as ex
    from oxforge import net

    def rel(a, b):
        b = np.asarray(b, np.float64)
        return float(np.max(np.abs(np.asarray(a, np.float64) - b)) /
                     max(np.max(np.abs(b)), 1e-30))

    rng = np.random.default_rng(3000 + seed)
    for case in range(6):
        S, H = int(rng.integers(2, 300)), int(rng.integers(8, 97))
        F, O = int(rng.integers(4, 257)), int(rng.integers(4, 81))
        norm = int(rng.choice([net.LAYER, net.RMS]))
        act = int(rng.integers(0, 4))
        bias, affine = bool(rng.random() < 0.6), bool(rng.random() < 0.6)
        kind = int(rng.choice([net.ENCODER_INFERENCE, net.DECODER_INFERENCE,
                               net.ENCODER_TRAINING]))
        streams = bool(rng.random() < 0.5) and kind != net.ENCODER_TRAINING
        chunked = bool(rng.random() < 0.5)
        say(f"seed {seed} case {case}: S={S} H={H} F={F} O={O} norm={norm} act={act} "
            f"bias={bias} affine={affine} kind={kind} streams={streams} chunked={chunked}")
        ps = int(rng.integers(0, 1 << 20))
        p = {"WQ": synth.xavier(H, H, ps), "WK": synth.xavier(H, H, ps + 1),
             "WV": synth.xavier(H, H, ps + 2), "POS": synth.xavier(S, H, ps + 3),
             "W1": synth.xavier(H, F, ps + 4), "W2": synth.xavier(F, H, ps + 5),
             "WO": synth.xavier(H, O, ps + 6)}
        for i, (k, n) in enumerate((("BQ", H), ("BK", H), ("BV", H), ("B1", F), ("B2", H),
                                    ("BO", O))):
            p[k] = synth.normal((n,), ps + 10 + i, 0.0, 0.1) if bias else None
        for i, k in enumerate(("G1", "G2")):
            p[k] = synth.normal((H,), ps + 20 + i, 1.0, 0.1) if affine else None
        for i, k in enumerate(("BE1", "BE2")):
            p[k] = (synth.normal((H,), ps + 22 + i, 0.0, 0.1)
                    if affine and norm == net.LAYER else None)
        X = synth.normal((S, H), ps + 30)
        T = net.Transformer(rt, p, S, H, F, O, norm, kind, streams, ffn_activation=act)
        if chunked:
            T.set_score_bytes(64 * S * 4)  # chunks of 64 query rows
        Y = T.forward(rt.array(X)).numpy()
        ref, cache = ex.transformer_forward(p, X, norm, act,
                                            causal=(kind == net.DECODER_INFERENCE))
        assert rel(Y, ref) <= 1e-4, "forward"
        if kind == net.ENCODER_TRAINING:
            dY = synth.normal((S, O), ps + 31)
            lr = np.float32(1e-3)
            dX = rt.empty((S, H))
            grads = T.backward(rt.array(dY), float(lr), dX, want_grads=True)
            rdX, rg = ex.transformer_backward(p, cache, dY, norm, act)
            assert rel(dX.numpy(), rdX) <= 1e-4, "dX"
            for k in net.TP_SLOTS:
                if rg.get(k) is None or p.get(k) is None:
                    continue
                g = grads[k].numpy()
                if k == "BK":  # zero in exact arithmetic (softmax shift invariance)
                    assert np.max(np.abs(g)) <= 1e-4 * max(np.max(np.abs(rg["BV"])), 1e-30)
                else:
                    assert rel(g, rg[k]) <= 1e-4, k
                assert np.array_equal(T.param(k), p[k] - lr * g), f"SGD update of {k}"
        T.close()


@pytest.mark.parametrize("seed", range(4))
def test_mlp_random_configs(rt, seed):
    """Random MLPs (mlp.rs:14-269): 1-5 layers of random widths, each
    activation, biases or none, with or without a residual range
    [start, end) (the input of layer start added to the output of layer
    end - 1, so the two widths match); inference output, and for the
    training executor the input gradient and the SGD identity of every
    weight and bias, against the f64 oracle."""
    from oracle import executors as ex
    from oxforge import net

    def rel(a, b):
        b = np.asarray(b, np.float64)
        return float(np.max(np.abs(np.asarray(a, np.float64) - b)) /
                     max(np.max(np.abs(b)), 1e-30))

    rng = np.random.default_rng(4000 + seed)
    for case in range(6):
        L = int(rng.integers(1, 6))
        dims = [int(rng.integers(1, 200)) for _ in range(L + 1)]
        res = None
        if L >= 1 and rng.random() < 0.5:
            start = int(rng.integers(0, L))
            end = int(rng.integers(start + 1, L + 1))
            dims[end] = dims[start]
            res = (start, end)
        rows = int(rng.integers(1, 300))
        ps = int(rng.integers(0, 1 << 20))
        layers = [(synth.xavier(dims[i], dims[i + 1], ps + i),
                   synth.normal((dims[i + 1],), ps + 50 + i, 0.0, 0.1) if rng.random() < 0.7 else None,
                   int(rng.integers(0, 4))) for i in range(L)]
        training = bool(rng.random() < 0.5)
        say(f"seed {seed} case {case}: dims={dims} res={res} rows={rows} training={training} "
            f"acts={[a for _, _, a in layers]}")
        X = synth.normal((rows, dims[0]), ps + 99)
        m = net.Mlp(rt, layers, res, training=training)
        Y = m.forward(rt.array(X)).numpy()
        ref, ins, pres = ex.mlp_forward(layers, X, res)
        assert rel(Y, ref) <= 1e-4, "forward"
        if training:
            dY = synth.normal((rows, dims[-1]), ps + 98)
            lr = np.float32(1e-2)
            dX = m.backward(rt.array(dY), float(lr)).numpy()
            rdX, dWs, dbs = ex.mlp_backward(layers, ins, pres, dY, res)
            assert rel(dX, rdX) <= 1e-4, "dX"
            for i, (W, b, _) in enumerate(layers):
                assert rel(m.param(i, 0), W - lr * dWs[i]) <= 1e-4, f"W{i}"
                if b is not None:
                    assert rel(m.param(i, 1), b - lr * dbs[i]) <= 1e-4, f"b{i}"
        m.close()
