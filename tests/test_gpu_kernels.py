"""GPU parity of every kernel behind the C ABI against the CPU oracle.

Bars:
  - transpose, copy, broadcast, binary ops, fills: bit-exact;
  - GEMM: max|C - C64| / max|C64| <= 1e-4 and componentwise
    |C - C64| / (|A| |B|) <= 1e-4 against an f64-accumulated oracle, and
    bit-exact where fp32 is exact in any summation order (small integers,
    permutations);
  - softmax and norms, forward and backward: <= 1e-5 absolute;
  - maps built on tanhf/expf: <= 2e-6 absolute + relative.
The full benchmark sizes are covered directly (row ops, transpose) or through
sampled rows checked against the f64 oracle (GEMM).
"""
import numpy as np
import pytest

import oxforge
import rowbounds as rb
from oxforge import synth
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL_ROW = 1e-5


_CU = []


def col_tols(rt, x, dy, aligned=True, out_aligned=True):
    """Per-column tolerances of the norm backward's dgamma and dbeta
    (LayerNorm) and dgamma (RMSNorm): max(1e-5, 2 x the rounding bound of
    the kernels' column-sum tree over the kernels' own f32 terms,
    rowbounds.layer_norm_param_bounds / rms_norm_param_bound)."""
    if not _CU:
        _CU.append(rt.props()["cu_count"])
    bg, bb = rb.layer_norm_param_bounds(x, dy, _CU[0], aligned=aligned, out_aligned=out_aligned)
    br = rb.rms_norm_param_bound(x, dy, _CU[0], aligned=aligned, out_aligned=out_aligned)
    return rb.tolerance(bg), rb.tolerance(bb), rb.tolerance(br)


def within_cols(got, ref, tol, what=""):
    err = np.abs(np.asarray(got, np.float64) - ref)
    assert np.all(err <= tol), (what, float(err.max()), float(tol[np.argmax(err - tol)]))
    return float(err.max()), float((err / tol).max())


def say(msg):
    print(f"[case] {msg}", flush=True)


def gemm_errors(C, ref64, A64abs_B64abs):
    err = np.abs(C.astype(np.float64) - ref64)
    rel_max = float(err.max() / max(np.abs(ref64).max(), 1e-30))
    comp = float((err / np.maximum(A64abs_B64abs, 1e-30)).max())
    return rel_max, comp


def op_a(A, ta):
    return A.T if ta else A


# ------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(256, 64, 128), (128, 128, 16), (1, 1, 1), (17, 33, 5),
                                   (100, 257, 63), (64, 64, 64), (384, 256, 512), (130, 70, 1000)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_shapes_vs_oracle(rt, M, N, K, ta, tb):
    say(f"gemm M={M} N={N} K={K} ta={ta} tb={tb}")
    A = synth.uniform((K, M) if ta else (M, K), 1 + M)
    B = synth.uniform((N, K) if tb else (K, N), 2 + N)
    dA, dB, dC = rt.array(A), rt.array(B), rt.empty((M, N))
    if ta or tb:
        rt.gemm_ex(dA, dB, dC, M, N, K, trans_a=ta, trans_b=tb)
    else:
        rt.gemm(dA, dB, dC, M, N, K)
    C = dC.numpy()
    ref = orc.gemm_f64(A, B, ta, tb)
    absprod = np.abs(op_a(A, ta)).astype(np.float64) @ np.abs(op_a(B, tb)).astype(np.float64)
    rel_max, comp = gemm_errors(C, ref, absprod)
    assert rel_max <= 1e-4 and comp <= 1e-4, (rel_max, comp)
    for d in (dA, dB, dC):
        d.recycle()


@pytest.mark.parametrize("M,N,K", [(64, 128, 65536), (33, 65, 40001)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_long_k_vs_oracle(rt, M, N, K, ta, tb):
    """Long reductions: 65536 (the unguarded tiles, 2048 slabs) and 40001
    (the guarded tile, a ragged last slab) products per output element,
    against the f64-accumulated oracle at the same bars."""
    say(f"gemm long K M={M} N={N} K={K} ta={ta} tb={tb}")
    A = synth.uniform((K, M) if ta else (M, K), 7)
    B = synth.uniform((N, K) if tb else (K, N), 8)
    dA, dB, dC = rt.array(A), rt.array(B), rt.empty((M, N))
    rt.gemm_ex(dA, dB, dC, M, N, K, trans_a=ta, trans_b=tb)
    ref = orc.gemm_f64(A, B, ta, tb)
    absprod = np.abs(op_a(A, ta)).astype(np.float64) @ np.abs(op_a(B, tb)).astype(np.float64)
    rel_max, comp = gemm_errors(dC.numpy(), ref, absprod)
    print(f"  long K {M}x{N}x{K}: rel_max {rel_max:.2e}, componentwise {comp:.2e}")
    assert rel_max <= 1e-4 and comp <= 1e-4, (rel_max, comp)
    for d in (dA, dB, dC):
        d.recycle()


def test_gemm_small_integers_bit_exact(rt):
    say("gemm small integers 512x384x4096")
    r = np.random.default_rng(0)
    M, N, K = 512, 384, 4096
    A = r.integers(-16, 17, (M, K)).astype(np.float32)
    B = r.integers(-16, 17, (K, N)).astype(np.float32)
    dA, dB, dC = rt.array(A), rt.array(B), rt.empty((M, N))
    rt.gemm(dA, dB, dC, M, N, K)
    exact = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(dC.numpy(), exact)


def test_gemm_permutation_bit_exact(rt):
    say("gemm permutation 256x256x256")
    A = synth.uniform((256, 256), 5)
    perm = np.random.default_rng(1).permutation(256)
    P = np.zeros((256, 256), np.float32)
    P[np.arange(256), perm] = 1.0
    dA, dP, dC = rt.array(A), rt.array(P), rt.empty((256, 256))
    rt.gemm(dA, dP, dC, 256, 256, 256)
    assert np.array_equal(dC.numpy(), A @ P)


def test_gemm_k_zero_writes_zeros(rt):
    say("gemm K=0")
    dA, dB, dC = rt.empty((0,)), rt.empty((0,)), rt.array(np.ones((8, 8), np.float32))
    rt.gemm(dA, dB, dC, 8, 8, 0)
    assert np.array_equal(dC.numpy(), np.zeros((8, 8), np.float32))


def test_gemm_short_slice_rejected(rt):
    dA, dB, dC = rt.empty((4, 4)), rt.empty((4, 4)), rt.empty((4, 3))
    with pytest.raises(oxforge.ForgeError) as e:
        rt.gemm(dA, dB, dC, 4, 4, 4)
    assert e.value.status == 1


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (8192, 1024, 4096)])
def test_gemm_full_size_sampled_rows(rt, M, N, K):
    say(f"gemm full size {M}x{N}x{K}")
    A = synth.uniform((M, K), 3)
    B = synth.uniform((K, N), 4)
    dA, dB, dC = rt.array(A), rt.array(B), rt.empty((M, N))
    rt.gemm(dA, dB, dC, M, N, K)
    C = dC.numpy()
    # One row in every 64-row band (at a different offset in each band) and
    # 64 columns spread over N, each against the f64 oracle: every row band
    # and every 64-column group of output tiles is checked somewhere.
    bands = M // 64
    rows = np.arange(bands) * 64 + (np.arange(bands) * 37) % 64
    ref = orc.gemm_f64(np.ascontiguousarray(A[rows]), B)
    absprod = np.abs(A[rows]).astype(np.float64) @ np.abs(B).astype(np.float64)
    rel_max, comp = gemm_errors(C[rows], ref, absprod)
    assert rel_max <= 1e-4 and comp <= 1e-4, (rel_max, comp)
    cols = np.arange(64) * (N // 64) + (np.arange(64) * 11) % (N // 64)
    Bc = np.ascontiguousarray(B[:, cols])
    ref = orc.gemm_f64(A, Bc)
    absprod = np.abs(A).astype(np.float64) @ np.abs(Bc).astype(np.float64)
    rel_max, comp = gemm_errors(np.ascontiguousarray(C[:, cols]), ref, absprod)
    print(f"  sampled rows and columns: max rel err {rel_max:.2e}, componentwise {comp:.2e}")
    assert rel_max <= 1e-4 and comp <= 1e-4, (rel_max, comp)
    # every tile was written: row sums against A @ (B @ 1) in f64
    ones = B.astype(np.float64).sum(axis=1)
    approx = A.astype(np.float64) @ ones
    assert np.allclose(C.astype(np.float64).sum(axis=1), approx, rtol=1e-3, atol=1e-1)
    for d in (dA, dB, dC):
        d.recycle()


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(256, 128, 64), (50, 70, 33), (256, 128, 2048)])
def test_gemm_epilogue_matches_unfused_bit_exact(rt, M, N, K, ta, tb):
    """Fused bias + residual + aux + activation + update equals the unfused
    launch sequence of Linear::affine_on/activate_on/learn_on bit for bit.
    256x128x2048 is computed as two K slices, so the split-K reduction's
    epilogue is covered too."""
    say(f"gemm epilogue M={M} N={N} K={K} ta={ta} tb={tb}")
    A = synth.uniform((K, M) if ta else (M, K), 7)
    B = synth.uniform((N, K) if tb else (K, N), 8)
    bias = synth.uniform((N,), 9)
    res = synth.uniform((M, N), 10)
    aux = synth.uniform((M, N), 11)
    W = synth.uniform((M, N), 12)
    dA, dB = rt.array(A), rt.array(B)
    dbias, dres, daux = rt.array(bias), rt.array(res), rt.array(aux)
    for act, mop in [(oxforge.ACT_IDENTITY, None), (oxforge.ACT_GELU, oxforge.MAP_GELU),
                     (oxforge.ACT_RELU, oxforge.MAP_RELU), (oxforge.ACT_SILU, oxforge.MAP_SILU)]:
        # unfused: product, then by-rows bias, residual, aux, activation
        dZ = rt.empty((M, N))
        rt.gemm_ex(dA, dB, dZ, M, N, K, trans_a=ta, trans_b=tb)
        rt.map(dZ, oxforge.MAP_SCALE, 0.5)
        rt.binary_assign_by_rows(dZ, dbias, M, N, oxforge.ADD)
        rt.binary_assign(dZ, dres, oxforge.ADD)
        rt.binary_assign(dZ, daux, oxforge.MUL)
        pre_ref = dZ.numpy()
        if mop is not None:
            rt.map(dZ, mop)
        y_ref = dZ.numpy()
        # fused
        dY, dPre = rt.empty((M, N)), rt.empty((M, N))
        rt.gemm_ex(dA, dB, dY, M, N, K, trans_a=ta, trans_b=tb, alpha=0.5, bias=dbias,
                   residual=dres, aux_mul=daux, pre_out=dPre, activation=act)
        assert np.array_equal(dPre.numpy(), pre_ref), act
        assert np.array_equal(dY.numpy(), y_ref), act
    # Z * act'(aux): the derivative step of Linear::backward fused.
    for act, dop in [(oxforge.ACT_GELU, oxforge.MAP_GELU_D), (oxforge.ACT_RELU, oxforge.MAP_RELU_D),
                     (oxforge.ACT_SILU, oxforge.MAP_SILU_D)]:
        dZ = rt.empty((M, N))
        rt.gemm_ex(dA, dB, dZ, M, N, K, trans_a=ta, trans_b=tb)
        dD = rt.array(aux)
        rt.map(dD, dop)
        rt.binary_assign(dZ, dD, oxforge.MUL)
        dY = rt.empty((M, N))
        rt.gemm_ex(dA, dB, dY, M, N, K, trans_a=ta, trans_b=tb, aux_mul=daux,
                   aux_activation=act)
        assert np.array_equal(dY.numpy(), dZ.numpy()), act
    # SGD update: W - lr * (A B), as learn_on scales then subtracts
    lr = 1e-3
    dW = rt.array(W)
    rt.gemm_ex(dA, dB, dW, M, N, K, trans_a=ta, trans_b=tb, update=True, update_scale=lr)
    dG = rt.empty((M, N))
    rt.gemm_ex(dA, dB, dG, M, N, K, trans_a=ta, trans_b=tb)
    rt.map(dG, oxforge.MAP_SCALE, lr)
    dW2 = rt.array(W)
    rt.binary_assign(dW2, dG, oxforge.SUB)
    assert np.array_equal(dW.numpy(), dW2.numpy())


# -------------------------------------------------------------- transpose
@pytest.mark.parametrize("rows,cols", [(64, 64), (128, 256), (17, 33), (1, 100), (100, 1),
                                       (65, 129), (0, 5), (192, 768), (256, 1280),
                                       (8192, 4096)])
def test_transpose_bit_exact(rt, rows, cols):
    say(f"transpose {rows}x{cols}")
    x = synth.uniform((rows, cols), rows + cols)
    dx, dt = rt.array(x), rt.empty((cols, rows))
    rt.transpose(dx, dt, rows, cols)
    t = dt.numpy()
    assert np.array_equal(t, x.T)
    if rows * cols:
        dback = rt.empty((rows, cols))
        rt.transpose(dt, dback, cols, rows)
        assert np.array_equal(dback.numpy(), x)


def test_transpose_unaligned_view(rt):
    say("transpose unaligned view")
    x = synth.uniform((1 + 40 * 24,), 3)
    dx = rt.array(x)
    v = dx.view(1, (40, 24))
    dt = rt.empty((24, 40))
    rt.transpose(v, dt, 40, 24)
    assert np.array_equal(dt.numpy(), x[1:].reshape(40, 24).T)


# ---------------------------------------------------------------- row ops
ROW_SHAPES = [(4096, 1024), (4096, 2048), (5, 1), (7, 3), (33, 63), (9, 100), (64, 256), (17, 1000),
              (8, 1025), (16, 2048), (8, 4096), (4, 5000), (3, 9000), (2, 65536)]


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
def test_softmax_fwd_bwd(rt, rows, cols):
    say(f"softmax {rows}x{cols}")
    x = synth.normal((rows, cols), 2)
    g = synth.normal((rows, cols), 3)
    dx = rt.array(x)
    rt.softmax_rows(dx, rows, cols)
    p = dx.numpy()
    assert np.max(np.abs(p - orc.softmax_rows(x))) <= TOL_ROW
    dp, dg, dd = rt.array(p), rt.array(g), rt.empty((rows, cols))
    rt.softmax_rows_bwd(dp, dg, dd, rows, cols)
    assert np.max(np.abs(dd.numpy() - orc.softmax_rows_backward(p, g))) <= TOL_ROW


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm_fwd_bwd(rt, rows, cols, affine):
    say(f"layer_norm {rows}x{cols} affine={affine}")
    x = synth.normal((rows, cols), 2)
    dy = synth.normal((rows, cols), 3)
    gam = synth.normal((cols,), 4, 1.0, 0.1) if affine else None
    bet = synth.normal((cols,), 5, 0.0, 0.1) if affine else None
    dgam = rt.array(gam) if affine else None
    dbet = rt.array(bet) if affine else None
    d = rt.array(x)
    rt.layer_norm(d, rows, cols, gamma=dgam, beta=dbet)
    assert np.max(np.abs(d.numpy() - orc.layer_norm(x, gam, bet))) <= TOL_ROW
    dX, dDY, dDX = rt.array(x), rt.array(dy), rt.empty((rows, cols))
    pg, pb = rt.empty((cols,)), rt.empty((cols,))
    rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg, dbeta=pb)
    rdx, rdg, rdb = orc.layer_norm_backward(x, dy, gam, want_params=True)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    # column sums over `rows` terms: the derived per-column bound
    tg, tb, _ = col_tols(rt, x, dy)
    eg, fg = within_cols(pg.numpy(), rdg, tg, "dgamma")
    eb, fb = within_cols(pb.numpy(), rdb, tb, "dbeta")
    print(f"  dgamma max abs err {eg:.2e} ({fg:.2f} of its tolerance, max |dgamma| "
          f"{np.max(np.abs(rdg)):.2e}), dbeta {eb:.2e} ({fb:.2f})")


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
@pytest.mark.parametrize("affine", [False, True])
def test_rms_norm_fwd_bwd(rt, rows, cols, affine):
    say(f"rms_norm {rows}x{cols} affine={affine}")
    x = synth.normal((rows, cols), 6)
    dy = synth.normal((rows, cols), 7)
    gam = synth.normal((cols,), 8, 1.0, 0.1) if affine else None
    dgam = rt.array(gam) if affine else None
    d = rt.array(x)
    rt.rms_norm(d, rows, cols, gamma=dgam)
    assert np.max(np.abs(d.numpy() - orc.rms_norm(x, gam))) <= TOL_ROW
    dX, dDY, dDX, pg = rt.array(x), rt.array(dy), rt.empty((rows, cols)), rt.empty((cols,))
    rt.rms_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg)
    rdx, rdg = orc.rms_norm_backward(x, dy, gam, want_params=True)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    _, _, tr = col_tols(rt, x, dy)
    er, fr = within_cols(pg.numpy(), rdg, tr, "rms dgamma")
    print(f"  rms dgamma max abs err {er:.2e} ({fr:.2f} of its tolerance)")


def test_row_ops_reduce_to_reference_at_unit_affine(rt):
    """gamma = 1, beta = 0 reproduces the reference (no-affine) kernels bit for bit."""
    say("unit affine")
    x = synth.normal((64, 1024), 9)
    ones, zeros = rt.array(np.ones(1024, np.float32)), rt.array(np.zeros(1024, np.float32))
    a, b = rt.array(x), rt.array(x)
    rt.layer_norm(a, 64, 1024)
    rt.layer_norm(b, 64, 1024, gamma=ones, beta=zeros)
    assert np.array_equal(a.numpy(), b.numpy())
    a, b = rt.array(x), rt.array(x)
    rt.rms_norm(a, 64, 1024)
    rt.rms_norm(b, 64, 1024, gamma=ones)
    assert np.array_equal(a.numpy(), b.numpy())


def test_row_ops_unaligned_views(rt):
    say("row ops unaligned views")
    x = synth.normal((1 + 12 * 40,), 10)
    d = rt.array(x)
    v = d.view(1, (12, 40))
    rt.softmax_rows(v, 12, 40)
    assert np.max(np.abs(v.numpy() - orc.softmax_rows(x[1:].reshape(12, 40)))) <= TOL_ROW


def test_norm_bwd_column_sums_across_launches(rt):
    """dgamma / dbeta: per-workgroup partial rows, then one final column-sum
    pass (float4 columns when the outputs are 16-byte aligned, scalar
    otherwise).  Launches of different grids in a row, requests of dgamma or
    dbeta alone and unaligned outputs must each match the oracle, and a
    repeated launch must reproduce its result bit for bit."""
    cols = 1024
    gam_h = synth.normal((cols,), 31, 1.0, 0.1)
    dgam = rt.array(gam_h)
    for rows in (4096, 8, 100, 1600, 4096, 1, 2056):
        say(f"norm bwd column sums rows={rows}")
        x, dy = synth.normal((rows, cols), 32 + rows), synth.normal((rows, cols), 33 + rows)
        dX, dDY, dDX = rt.array(x), rt.array(dy), rt.empty((rows, cols))
        tg, tb, tr = col_tols(rt, x, dy)
        ug_tg, ug_tb, _ = col_tols(rt, x, dy, out_aligned=False)
        rdx, rdg, rdb = orc.layer_norm_backward(x, dy, gam_h, want_params=True)
        runs = []
        for _ in range(2):
            pg, pb = rt.empty((cols,)), rt.empty((cols,))
            rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg, dbeta=pb)
            runs.append((pg.numpy(), pb.numpy()))
        assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1])
        within_cols(runs[0][0], rdg, tg, "dgamma")
        within_cols(runs[0][1], rdb, tb, "dbeta")
        assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
        only_g, only_b = rt.empty((cols,)), rt.empty((cols,))
        rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=only_g)
        rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dbeta=only_b)
        assert np.array_equal(only_g.numpy(), runs[0][0])
        assert np.array_equal(only_b.numpy(), runs[0][1])
        # dgamma / dbeta not 16-byte aligned: the separate column-sum pass.
        ub = rt.empty((2 * cols + 2,))
        ug, ubt = ub.view(1, (cols,)), ub.view(cols + 2, (cols,))
        rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=ug, dbeta=ubt)
        within_cols(ug.numpy(), rdg, ug_tg, "unaligned dgamma")
        within_cols(ubt.numpy(), rdb, ug_tb, "unaligned dbeta")
        rdx, rdg = orc.rms_norm_backward(x, dy, gam_h, want_params=True)
        rg = rt.empty((cols,))
        rt.rms_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=rg)
        within_cols(rg.numpy(), rdg, tr, "rms dgamma")
        assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW


# Aligned widths with cols % 4 == 0 that are not a multiple of 256 leave
# lanes past the row end in the register kernels (v8, v16 and their
# partial instances read gamma per use).  gamma sits in a buffer whose tail
# past cols holds NaN: a kernel that read or used gamma beyond the row would
# turn the row's results into NaN.
MASKED_LANE_SHAPES = [(8, 1028), (8, 1540), (4, 2052), (4, 3000), (64, 1028), (300, 1540)]


@pytest.mark.parametrize("rows,cols", MASKED_LANE_SHAPES)
@pytest.mark.parametrize("params", [False, True])
def test_norms_masked_lanes_read_no_gamma_past_row(rt, rows, cols, params):
    say(f"norms masked lanes {rows}x{cols} params={params}")
    pad = 4096
    x = synth.normal((rows, cols), 41 + cols)
    dy = synth.normal((rows, cols), 42 + cols)
    gam = synth.normal((cols,), 43, 1.0, 0.1)
    bet = synth.normal((cols,), 44, 0.0, 0.1)
    gbuf = rt.array(np.concatenate([gam, np.full(pad, np.nan, np.float32)]))
    bbuf = rt.array(np.concatenate([bet, np.full(pad, np.nan, np.float32)]))
    dgam, dbet = gbuf.view(0, (cols,)), bbuf.view(0, (cols,))
    tg, tb, tr = col_tols(rt, x, dy)

    d = rt.array(x)
    rt.layer_norm(d, rows, cols, gamma=dgam, beta=dbet)
    assert np.max(np.abs(d.numpy() - orc.layer_norm(x, gam, bet))) <= TOL_ROW
    d = rt.array(x)
    rt.rms_norm(d, rows, cols, gamma=dgam)
    assert np.max(np.abs(d.numpy() - orc.rms_norm(x, gam))) <= TOL_ROW

    dX, dDY, dDX = rt.array(x), rt.array(dy), rt.empty((rows, cols))
    rdx, rdg, rdb = orc.layer_norm_backward(x, dy, gam, want_params=True)
    pg, pb = (rt.empty((cols,)), rt.empty((cols,))) if params else (None, None)
    rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg, dbeta=pb)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    if params:
        within_cols(pg.numpy(), rdg, tg, "dgamma")
        within_cols(pb.numpy(), rdb, tb, "dbeta")

    rdx, rdg = orc.rms_norm_backward(x, dy, gam, want_params=True)
    rg = rt.empty((cols,)) if params else None
    rt.rms_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=rg)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    if params:
        within_cols(rg.numpy(), rdg, tr, "rms dgamma")


# Outputs of 16M floats (64 MiB) and more are stored non-temporally; the
# shapes above stay below that, these two tests cover the other path.
NT_ROWS, NT_COLS = 16384, 1024


@pytest.mark.parametrize("affine", [False, True])
def test_row_kernels_at_nontemporal_size(rt, affine):
    rows, cols = NT_ROWS, NT_COLS
    say(f"row kernels {rows}x{cols} affine={affine}")
    x, dy = synth.normal((rows, cols), 21), synth.normal((rows, cols), 22)
    gam = synth.normal((cols,), 23, 1.0, 0.1) if affine else None
    bet = synth.normal((cols,), 24, 0.0, 0.1) if affine else None
    dgam = rt.array(gam) if affine else None
    dbet = rt.array(bet) if affine else None
    tg, tb, tr = col_tols(rt, x, dy)
    d = rt.array(x)
    rt.softmax_rows(d, rows, cols)
    p = d.numpy()
    assert np.max(np.abs(p - orc.softmax_rows(x))) <= TOL_ROW
    dp, dg, dd = rt.array(p), rt.array(dy), rt.empty((rows, cols))
    rt.softmax_rows_bwd(dp, dg, dd, rows, cols)
    assert np.max(np.abs(dd.numpy() - orc.softmax_rows_backward(p, dy))) <= TOL_ROW
    d = rt.array(x)
    rt.layer_norm(d, rows, cols, gamma=dgam, beta=dbet)
    assert np.max(np.abs(d.numpy() - orc.layer_norm(x, gam, bet))) <= TOL_ROW
    dX, dDY, dDX = rt.array(x), rt.array(dy), rt.empty((rows, cols))
    pg, pb = rt.empty((cols,)), rt.empty((cols,))
    rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg, dbeta=pb)
    rdx, rdg, rdb = orc.layer_norm_backward(x, dy, gam, want_params=True)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    within_cols(pg.numpy(), rdg, tg, "dgamma")
    within_cols(pb.numpy(), rdb, tb, "dbeta")
    d = rt.array(x)
    rt.rms_norm(d, rows, cols, gamma=dgam)
    assert np.max(np.abs(d.numpy() - orc.rms_norm(x, gam))) <= TOL_ROW
    rt.rms_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg)
    rdx, rdg = orc.rms_norm_backward(x, dy, gam, want_params=True)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    within_cols(pg.numpy(), rdg, tr, "rms dgamma")


def test_layer_norm_forward_both_parameter_paths(rt):
    """LayerNorm forward below 2^24 elements stages gamma/beta in LDS once per
    workgroup, from 2^24 on each wave loads them: [16383, 1024] and
    [16384, 1024] take one path each.  Both against the oracle, and the rows
    they share bit for bit (only where gamma/beta are read from differs)."""
    cols = 1024
    x = synth.normal((16384, cols), 71)
    gam, bet = synth.normal((cols,), 72, 1.0, 0.1), synth.normal((cols,), 73, 0.0, 0.1)
    dgam, dbet = rt.array(gam), rt.array(bet)
    out = {}
    for rows in (16383, 16384):
        say(f"layer norm forward {rows}x{cols}")
        d = rt.array(x[:rows])
        rt.layer_norm(d, rows, cols, gamma=dgam, beta=dbet)
        out[rows] = d.numpy()
        assert np.max(np.abs(out[rows] - orc.layer_norm(x[:rows], gam, bet))) <= TOL_ROW
        d.recycle()
    assert np.array_equal(out[16383], out[16384][:16383])


@pytest.mark.parametrize("rows,cols", [(65536, 1024), (65537, 1000)])
def test_norm_bwd_partials_at_scale_four_wave_instance(rt, rows, cols):
    """[65536, 1024] takes the four-wave partial instance (_p4: 256 rows per
    CU and more; two workgroups per CU for the LayerNorm backward), and so
    does [65537, 1000] with a ragged last row block and masked lanes.  dx
    against the oracle on every row; dgamma / dbeta (sums over the rows)
    within the derived column-sum tolerance (col_tols), the measured error
    and its share of the tolerance printed."""
    say(f"norm bwd partials {rows}x{cols}")
    x, dy = synth.normal((rows, cols), 51), synth.normal((rows, cols), 52)
    gam = synth.normal((cols,), 53, 1.0, 0.1)
    dgam = rt.array(gam)
    dX, dDY, dDX = rt.array(x), rt.array(dy), rt.empty((rows, cols))
    pg, pb = rt.empty((cols,)), rt.empty((cols,))
    tg, tb, tr = col_tols(rt, x, dy)
    rt.layer_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg, dbeta=pb)
    rdx, rdg, rdb = orc.layer_norm_backward(x, dy, gam, want_params=True)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    eg, fg = within_cols(pg.numpy(), rdg, tg, "dgamma")
    eb, fb = within_cols(pb.numpy(), rdb, tb, "dbeta")
    print(f"  LN dgamma max abs err {eg:.2e} ({fg:.2f} of its tolerance, max |dgamma| "
          f"{np.max(np.abs(rdg)):.2e}), dbeta {eb:.2e} ({fb:.2f})")
    rt.rms_norm_bwd(dX, dDY, dDX, rows, cols, gamma=dgam, dgamma=pg)
    rdx, rdg = orc.rms_norm_backward(x, dy, gam, want_params=True)
    assert np.max(np.abs(dDX.numpy() - rdx)) <= TOL_ROW
    er, fr = within_cols(pg.numpy(), rdg, tr, "rms dgamma")
    print(f"  RMS dgamma max abs err {er:.2e} ({fr:.2f} of its tolerance)")
    for d in (dgam, dX, dDY, dDX, pg, pb):
        d.recycle()


@pytest.mark.parametrize("rows,cols", [(4096, 2048), (300, 1024), (600, 33), (513, 64), (7, 5),
                                       (0, 16)])
def test_sum_cols_sgd_matches_separate_launches(rt, rows, cols):
    """forge_sum_cols_sgd (column sums and the bias SGD step in the final
    pass) against forge_sum_cols then forge_sgd_update: bit for bit, with
    and without the sums kept, with and without the parameter."""
    say(f"sum_cols_sgd {rows}x{cols}")
    m = synth.normal((max(rows, 1), cols), 61)[:rows]
    b = synth.normal((cols,), 62)
    lr = 1e-3
    dm = rt.array(np.ascontiguousarray(m)) if rows else rt.empty((0,))
    ref_s, ref_p = rt.empty((cols,)), rt.array(b)
    rt.sum_cols(dm, ref_s, rows, cols)
    rt.sgd_update(ref_p, ref_s, lr)
    for keep, upd in ((True, True), (False, True), (True, False)):
        out = rt.array(np.full(cols, np.nan, np.float32)) if keep else None
        par = rt.array(b) if upd else None
        rt.sum_cols_sgd(dm, rows, cols, lr, out=out, param=par)
        if keep:
            assert np.array_equal(out.numpy(), ref_s.numpy())
        if upd:
            assert np.array_equal(par.numpy(), ref_p.numpy())


@pytest.mark.parametrize("rows,cols", [(4096, 1024), (4096, 2048), (65536, 1024), (33, 1001),
                                       (0, 64)])
def test_norm_bwd_sgd_matches_separate_launches(rt, rows, cols):
    """forge_layer_norm_bwd_sgd / forge_rms_norm_bwd_sgd against the norm
    backward then forge_sgd_update on gamma and beta: dx, the gradients and
    the updated parameters bit for bit (dx uses the gamma from before the
    step)."""
    say(f"norm bwd sgd {rows}x{cols}")
    x = synth.normal((max(rows, 1), cols), 63)[:rows]
    dy = synth.normal((max(rows, 1), cols), 64)[:rows]
    gam, bet = synth.normal((cols,), 65, 1.0, 0.1), synth.normal((cols,), 66, 0.0, 0.1)
    lr = 1e-3
    n = rows * cols
    dX = rt.array(np.ascontiguousarray(x)) if n else rt.empty((0,))
    dDY = rt.array(np.ascontiguousarray(dy)) if n else rt.empty((0,))
    # reference: separate launches
    g0, b0 = rt.array(gam), rt.array(bet)
    rdx, rdg, rdb = rt.empty((max(n, 1),)), rt.empty((cols,)), rt.empty((cols,))
    rt.layer_norm_bwd(dX, dDY, rdx, rows, cols, gamma=g0, dgamma=rdg, dbeta=rdb)
    rt.sgd_update(g0, rdg, lr)
    rt.sgd_update(b0, rdb, lr)
    g1, b1 = rt.array(gam), rt.array(bet)
    fdx, fdg, fdb = rt.empty((max(n, 1),)), rt.empty((cols,)), rt.empty((cols,))
    rt.layer_norm_bwd_sgd(dX, dDY, fdx, rows, cols, lr, gamma=g1, beta=b1, dgamma=fdg, dbeta=fdb)
    assert np.array_equal(fdx.numpy()[:n], rdx.numpy()[:n])
    for u, v in ((fdg, rdg), (fdb, rdb), (g1, g0), (b1, b0)):
        assert np.array_equal(u.numpy(), v.numpy())
    # the step alone, no gradient outputs
    g2, b2 = rt.array(gam), rt.array(bet)
    rt.layer_norm_bwd_sgd(dX, dDY, fdx, rows, cols, lr, gamma=g2, beta=b2)
    assert np.array_equal(g2.numpy(), g0.numpy()) and np.array_equal(b2.numpy(), b0.numpy())
    # RMSNorm
    g0 = rt.array(gam)
    rt.rms_norm_bwd(dX, dDY, rdx, rows, cols, gamma=g0, dgamma=rdg)
    rt.sgd_update(g0, rdg, lr)
    g1 = rt.array(gam)
    rt.rms_norm_bwd_sgd(dX, dDY, fdx, rows, cols, lr, gamma=g1, dgamma=fdg)
    assert np.array_equal(fdx.numpy()[:n], rdx.numpy()[:n])
    assert np.array_equal(fdg.numpy(), rdg.numpy()) and np.array_equal(g1.numpy(), g0.numpy())


@pytest.mark.parametrize("rows,cols", [(513, 64), (300, 500), (257, 1000), (4096, 2048),
                                       (96, 4096), (65536, 1024), (77, 1001), (0, 64), (7, 0)])
def test_norm_bwd_row_dot(rt, rows, cols):
    """forge_layer_norm_bwd_sgd_dot / forge_rms_norm_bwd_sgd_dot (the
    attention backward's softmax row term): dx, the gradients and the
    updated parameters bit for bit those of the _sgd entry points, with
    gamma/beta (the column-partial instances) and without (the plain ones);
    dot[r] = s * sum_c dx[r,c] (x[r,c] - sub[r,c]) from the returned dx within
    (cols + 8) u |s| sum_c |dx| |x - sub| of the f64 value (one rounding for
    x - sub, one per product, at most cols - 1 in the sum, one for s), and
    nothing written past `rows`.  The widths take every register instance
    (1, 2, 4, 8 and 16 float4 per lane; the four-wave partial instance at
    65536 rows) and the looping path (1001 columns, and 4096 with gamma);
    rows of no columns have a zero dot."""
    say(f"norm bwd row dot {rows}x{cols}")
    u = 2.0 ** -24
    x = synth.normal((max(rows, 1), cols), 163)[:rows]
    dy = synth.normal((max(rows, 1), cols), 164)[:rows]
    sub = synth.normal((max(rows, 1), cols), 167)[:rows]
    gam, bet = synth.normal((cols,), 165, 1.0, 0.1), synth.normal((cols,), 166, 0.0, 0.1)
    lr, s = 1e-3, 1.0 / np.sqrt(max(cols, 1))
    n = rows * cols
    dev = (lambda a: rt.array(np.ascontiguousarray(a))) if n else (lambda a: rt.empty((0,)))
    dX, dDY, dSUB = dev(x), dev(dy), dev(sub)
    rdx, fdx = rt.empty((max(n, 1),)), rt.empty((max(n, 1),))
    for norm in ("layer", "rms"):
        for params in (True, False):
            say(f"  {norm} params={params}")
            g0, b0, g1, b1 = (rt.array(v) for v in (gam, bet, gam, bet))
            rdg, rdb, fdg, fdb = (rt.empty((cols,)) for _ in range(4))
            dot = rt.array(np.full(rows + 1, np.nan, np.float32))
            if norm == "layer":
                kw = dict(gamma=g0, beta=b0, dgamma=rdg, dbeta=rdb) if params else {}
                rt.layer_norm_bwd_sgd(dX, dDY, rdx, rows, cols, lr, **kw)
                kw = dict(gamma=g1, beta=b1, dgamma=fdg, dbeta=fdb) if params else {}
                rt.layer_norm_bwd_sgd_dot(dX, dDY, fdx, dSUB, dot, rows, cols, lr, dot_scale=s,
                                          **kw)
            else:
                kw = dict(gamma=g0, dgamma=rdg) if params else {}
                rt.rms_norm_bwd_sgd(dX, dDY, rdx, rows, cols, lr, **kw)
                kw = dict(gamma=g1, dgamma=fdg) if params else {}
                rt.rms_norm_bwd_sgd_dot(dX, dDY, fdx, dSUB, dot, rows, cols, lr, dot_scale=s,
                                        **kw)
            got_dx = fdx.numpy()[:n]
            assert np.array_equal(got_dx, rdx.numpy()[:n])
            if params:
                for a, b in ((fdg, rdg), (g1, g0)) + (((fdb, rdb), (b1, b0))
                                                      if norm == "layer" else ()):
                    assert np.array_equal(a.numpy(), b.numpy())
            got = dot.numpy()
            assert np.isnan(got[rows])
            if rows:
                d64 = got_dx.reshape(rows, cols).astype(np.float64)
                w = x.astype(np.float64) - sub.astype(np.float64)
                ref = s * (d64 * w).sum(axis=1)
                bound = (cols + 8) * u * s * (np.abs(d64) * np.abs(w)).sum(axis=1)
                err = np.abs(got[:rows] - ref)
                assert np.all(err <= bound), float(np.max(err / bound))


def test_norm_bwd_row_dot_rejects_overlaps(rt):
    """The row dot's operands: sub may not overlap dx (not even be it), nor
    dot any matrix operand."""
    rows, cols = 64, 256
    x, dy = rt.array(synth.normal((rows, cols), 1)), rt.array(synth.normal((rows, cols), 2))
    sub = rt.array(synth.normal((rows, cols), 3))
    big = rt.empty((rows * cols + rows,))
    dx = big.view(0, (rows, cols))
    for args in ((sub, big.view(cols, (rows,))),            # dot inside dx
                 (big.view(rows, (rows, cols)), rt.empty((rows,))),  # sub across dx
                 (dx, rt.empty((rows,))),                    # sub is dx
                 (sub, sub.view(5, (rows,)))):               # dot inside sub
        with pytest.raises(oxforge.ForgeError):
            rt.layer_norm_bwd_sgd_dot(x, dy, dx, args[0], args[1], rows, cols, 1e-3)
        with pytest.raises(oxforge.ForgeError):
            rt.rms_norm_bwd_sgd_dot(x, dy, dx, args[0], args[1], rows, cols, 1e-3)


# ------------------------------------------------------------ elementwise
OPS = [(oxforge.ADD, np.add), (oxforge.SUB, np.subtract), (oxforge.MUL, np.multiply),
       (oxforge.DIV, np.divide)]


def test_streaming_kernels_at_nontemporal_size(rt):
    """Binary ops, maps, SGD and the row broadcast stay bit-exact on the
    non-temporal store path."""
    rows, cols = NT_ROWS, NT_COLS
    n = rows * cols
    say(f"streaming kernels n={n}")
    a, b = synth.normal((n,), 11), synth.normal((n,), 12)
    da, db, do = rt.array(a), rt.array(b), rt.empty((n,))
    rt.binary(da, db, do, oxforge.ADD)
    assert np.array_equal(do.numpy(), a + b)
    rt.binary_assign(da, db, oxforge.MUL)
    assert np.array_equal(da.numpy(), a * b)
    rt.map(db, oxforge.MAP_SCALE, 0.37)
    assert np.array_equal(db.numpy(), np.float32(0.37) * b)
    dp, dgr = rt.array(a), rt.array(b)
    rt.sgd_update(dp, dgr, 0.01)
    assert np.array_equal(dp.numpy(), a - np.float32(0.01) * b)
    row = synth.normal((cols,), 13)
    dm = rt.array(a.reshape(rows, cols))
    rt.binary_assign_by_rows(dm, rt.array(row), rows, cols, oxforge.ADD)
    assert np.array_equal(dm.numpy(), a.reshape(rows, cols) + row[None, :])


@pytest.mark.parametrize("op,fn", OPS)
@pytest.mark.parametrize("n", [4096 * 1024, 1, 7, 1001])
def test_binary_bit_exact(rt, op, fn, n):
    say(f"binary op={op} n={n}")
    a = synth.normal((n,), 1)
    b = synth.normal((n,), 2)
    da, db, do = rt.array(a), rt.array(b), rt.empty((n,))
    rt.binary(da, db, do, op)
    assert np.array_equal(do.numpy(), fn(a, b))
    rt.binary_assign(da, db, op)
    assert np.array_equal(da.numpy(), fn(a, b))


def test_binary_unaligned_bit_exact(rt):
    say("binary unaligned")
    a = synth.normal((1001,), 1)
    b = synth.normal((1001,), 2)
    da, db, do = rt.array(a), rt.array(b), rt.empty((1001,))
    rt.binary(da.view(1, (1000,)), db.view(1, (1000,)), do.view(1, (1000,)), oxforge.MUL)
    assert np.array_equal(do.numpy()[1:], a[1:] * b[1:])


# One row per grid y index up to 65535; (70001, 8) and (65536, 12) also
# take the loop over further rows (vector and scalar instances).
@pytest.mark.parametrize("op,fn", OPS)
@pytest.mark.parametrize("rows,cols", [(4096, 1024), (3, 5), (70, 33), (1, 4), (70001, 8),
                                       (65536, 12), (65537, 7)])
def test_by_rows_bit_exact(rt, op, fn, rows, cols):
    say(f"by_rows op={op} {rows}x{cols}")
    m = synth.normal((rows, cols), 3)
    row = synth.normal((cols,), 4)
    dm, dr = rt.array(m), rt.array(row)
    rt.binary_assign_by_rows(dm, dr, rows, cols, op)
    assert np.array_equal(dm.numpy(), fn(m, row[None, :]))


EXACT_MAPS = [(oxforge.MAP_SCALE, 0.37), (oxforge.MAP_ADD, -1.25), (oxforge.MAP_HALF_SQ, 0.0),
              (oxforge.MAP_RELU, 0.0), (oxforge.MAP_RELU_D, 0.0), (oxforge.MAP_IDENTITY, 0.0)]
TRANS_MAPS = [(oxforge.MAP_GELU, 0.0), (oxforge.MAP_GELU_D, 0.0), (oxforge.MAP_SILU, 0.0),
              (oxforge.MAP_SILU_D, 0.0), (oxforge.MAP_EXP_SHIFT, 0.75)]


@pytest.mark.parametrize("op,p0", EXACT_MAPS + TRANS_MAPS)
def test_maps(rt, op, p0):
    say(f"map op={op}")
    x = synth.normal((4096 * 1024 + 3,), 5, 0.0, 2.0)
    d = rt.array(x)
    rt.map(d, op, p0)
    ref = orc.map_(x, op, p0)
    if (op, p0) in EXACT_MAPS:
        assert np.array_equal(d.numpy(), ref)
    else:
        y = d.numpy()
        assert np.all(np.abs(y - ref) <= 2e-6 + 2e-6 * np.abs(ref))


# Column sums take one pass up to 512 rows and two passes above: (512, 64)
# and (513, 64) sit on either side, (600, 33) is the unaligned two-pass path.
# The final pass reads float4 columns, 16 per workgroup, when cols % 4 == 0:
# (200, 36), (70, 1000) and (257, 20) leave a partial last workgroup.
@pytest.mark.parametrize("rows,cols", [(4096, 1024), (3, 7), (300, 33), (600, 33), (512, 64),
                                       (513, 64), (1, 1), (4096, 8192), (200, 36), (70, 1000),
                                       (257, 20), (1, 4)])
def test_sum_rows_cols(rt, rows, cols):
    say(f"sum rows/cols {rows}x{cols}")
    m = np.random.default_rng(rows).integers(-50, 51, (rows, cols)).astype(np.float32)
    dm, dr, dc = rt.array(m), rt.empty((rows,)), rt.empty((cols,))
    rt.sum_rows(dm, dr, rows, cols)
    rt.sum_cols(dm, dc, rows, cols)
    # integer inputs: every partial sum is exact, so any order is bit-exact
    assert np.array_equal(dr.numpy(), m.astype(np.int64).sum(axis=1).astype(np.float32))
    assert np.array_equal(dc.numpy(), m.astype(np.int64).sum(axis=0).astype(np.float32))
    mf = synth.normal((rows, cols), 6)
    dm2 = rt.array(mf)
    rt.sum_cols(dm2, dc, rows, cols)
    rt.sum_rows(dm2, dr, rows, cols)
    within_cols(dc.numpy(), orc.sum_cols(mf), rb.tolerance(rb.sum_cols_bound(mf)), "sum_cols")
    assert np.allclose(dr.numpy(), orc.sum_rows(mf), atol=1e-5 * np.sqrt(cols) + 1e-6)


# The float4 first pass of the column sums (more than 512 rows, 16-byte
# aligned float4 columns and outputs): partial last column groups (100, 1500
# and 2052 columns), a short last chunk (1000 rows), four columns, a single
# chunk that stores the sums itself (65600 columns), and the tall shapes.
# Repeated calls, and calls on forked streams with their own workspaces,
# agree bit for bit.
@pytest.mark.parametrize("rows,cols", [(1000, 100), (513, 4), (520, 65600), (65536, 1024),
                                       (4096, 2048), (700, 1500), (2000, 2052), (8192, 1024),
                                       (8193, 1024)])
def test_sum_cols_float4_first_pass(rt, rows, cols):
    say(f"sum_cols float4 first pass {rows}x{cols}")
    mf = synth.normal((rows, cols), 9)
    dm = rt.array(mf)
    first = rt.empty((cols,))
    rt.sum_cols(dm, first, rows, cols)
    ref = first.numpy()
    within_cols(ref, orc.sum_cols(mf), rb.tolerance(rb.sum_cols_bound(mf)), "sum_cols")
    out = rt.empty((cols,))
    for _ in range(3):
        rt.sum_cols(dm, out, rows, cols)
        assert np.array_equal(out.numpy(), ref)
    streams = rt.streams_create(2)
    outs = [rt.empty((cols,)) for _ in streams]
    rt.streams_fork(streams)
    for s, o in zip(streams, outs):
        rt.sum_cols(dm, o, rows, cols, stream=s)
        rt.sum_cols(dm, o, rows, cols, stream=s)
    rt.streams_join(streams)
    for o in outs:
        assert np.array_equal(o.numpy(), ref)
    # the SGD form writes the same sums and steps the parameter with them
    par0 = synth.normal((cols,), 10)
    par = rt.array(par0)
    rt.sum_cols_sgd(dm, rows, cols, 0.25, out=out, param=par)
    assert np.array_equal(out.numpy(), ref)
    assert np.array_equal(par.numpy(), par0 - np.float32(0.25) * ref)


@pytest.mark.parametrize("n", [1, 1000, 4096 * 1024, 10_000_019])
def test_reduce_sum_max(rt, n):
    say(f"reduce n={n}")
    x = np.random.default_rng(n).integers(-1000, 1001, n).astype(np.float32)
    dx, out = rt.array(x), rt.empty((1,))
    rt.reduce_sum(dx, out)
    assert out.numpy()[0] == float(x.astype(np.int64).sum())
    rt.reduce_max(dx, out)
    assert out.numpy()[0] == x.max()


@pytest.mark.parametrize("n", [5, 4096 * 1024 + 1])
def test_reduce_sum_max_unaligned_view(rt, n):
    """The scalar reduction path: a view that starts one float past a
    16-byte boundary (integer values, so every order is exact)."""
    say(f"reduce unaligned view n={n}")
    x = np.random.default_rng(n).integers(-1000, 1001, n).astype(np.float32)
    base = rt.empty((n + 1,))
    dx = base.view(1, (n,))
    dx.upload(x)
    out = rt.empty((1,))
    rt.reduce_sum(dx, out)
    assert out.numpy()[0] == float(x.astype(np.int64).sum())
    rt.reduce_max(dx, out)
    assert out.numpy()[0] == x.max()
    rt.map_sum(dx, out, oxforge.MAP_IDENTITY)
    assert out.numpy()[0] == float(x.astype(np.int64).sum())


@pytest.mark.parametrize("op,p0", EXACT_MAPS + TRANS_MAPS)
@pytest.mark.parametrize("n", [0, 1, 1001, 4096 * 1024 + 3])
def test_map_sum(rt, op, p0, n):
    """forge_map_sum (DeviceSpan::map_sum, span.rs:144-149 -> reduction.rs:
    43-91) against the f64 sum of the oracle's per-element map: within 1e-6
    of the sum of magnitudes (f32 accumulation over n terms in a fixed tree
    order).  Short integer-valued inputs with the exact functors are
    bit-exact.  An empty span sums to 0."""
    say(f"map_sum op={op} n={n}")
    x = synth.normal((n,), 7, 0.0, 2.0)
    dx, out = rt.array(x), rt.array(np.full((1,), np.nan, np.float32))
    rt.map_sum(dx, out, op, p0)
    mapped = orc.map_(x, op, p0).astype(np.float64) if n else np.zeros(0)
    got = float(out.numpy()[0])
    assert abs(got - mapped.sum()) <= 1e-6 * max(1.0, np.abs(mapped).sum()), (got, mapped.sum())
    # Short integer-valued spans: every partial sum is exact in f32.
    if (op, p0) in EXACT_MAPS and op != oxforge.MAP_SCALE and 0 < n <= 1001:
        xi = np.random.default_rng(n).integers(-30, 31, n).astype(np.float32)
        dx.upload(xi)
        rt.map_sum(dx, out, op, p0)
        exact = orc.map_(xi, op, p0).astype(np.float64).sum()
        assert float(out.numpy()[0]) == exact


def test_empty_shapes_and_oversized_dimensions(rt):
    """Zero rows, zero columns and zero-length spans launch nothing harmful
    and leave the reference's identities: column sums of no rows (and
    dgamma / dbeta of no rows) are zero, the full sum of an empty span is 0
    and its max f32::MIN (span.rs:302-321, as the oracle's pins check).
    Dimensions beyond 2^31 - 1 are refused before any launch."""
    say("empty shapes")
    cols = 64
    buf = rt.array(np.full(4 * cols, 7.0, np.float32))
    empty = rt.empty((0,))
    gam = rt.array(np.ones(cols, np.float32))
    for rows, c in ((0, cols), (5, 0), (0, 0)):
        rt.softmax_rows(empty, rows, c)
        rt.layer_norm(empty, rows, c, gamma=gam)
        rt.rms_norm(empty, rows, c, gamma=gam)
        rt.softmax_rows_bwd(empty, empty, empty, rows, c)
    dg, db = rt.array(np.full(cols, 3.0, np.float32)), rt.array(np.full(cols, 3.0, np.float32))
    rt.layer_norm_bwd(empty, empty, empty, 0, cols, gamma=gam, dgamma=dg, dbeta=db)
    assert np.all(dg.numpy() == 0) and np.all(db.numpy() == 0)
    dg2 = rt.array(np.full(cols, 3.0, np.float32))
    rt.rms_norm_bwd(empty, empty, empty, 0, cols, gamma=gam, dgamma=dg2)
    assert np.all(dg2.numpy() == 0)
    sc = rt.array(np.full(cols, 3.0, np.float32))
    rt.sum_cols(empty, sc, 0, cols)
    assert np.all(sc.numpy() == 0)
    rt.sum_rows(empty, sc, 0, cols)
    out = rt.empty((1,))
    rt.reduce_sum(empty, out, n=0)
    assert out.numpy()[0] == 0.0
    rt.reduce_max(empty, out, n=0)
    assert out.numpy()[0] == np.finfo(np.float32).min
    rt.binary(buf, buf, buf, oxforge.ADD, n=0)
    rt.map(buf, oxforge.MAP_SCALE, 2.0, n=0)
    rt.transpose(empty, empty, 0, cols)
    rt.gemm(empty, buf, empty, 0, 8, 8)
    rt.gemm(buf, empty, empty, 8, 0, 8)
    rt.sync()
    assert np.all(buf.numpy() == 7.0)  # nothing was written
    big = 1 << 31
    for fn in (lambda: rt.softmax_rows(buf, big, 1), lambda: rt.layer_norm(buf, 1, big),
               lambda: rt.sum_rows(buf, buf, big, 1), lambda: rt.sum_cols(buf, buf, 1, big),
               lambda: rt.transpose(buf, buf, big, 1), lambda: rt.gemm(buf, buf, buf, big, 1, 1)):
        with pytest.raises(oxforge.ForgeError) as e:
            fn()
        assert e.value.status == 1


def test_fills_and_causal_mask(rt):
    say("fills")
    d = rt.empty((1000,))
    rt.fill_seq(d, True)
    assert np.array_equal(d.numpy(), orc.fill_seq(1000, True))
    rt.fill_seq(d, False)
    assert np.array_equal(d.numpy(), orc.fill_seq(1000, False))
    rt.fill(d, 2.5)
    assert np.all(d.numpy() == 2.5)
    z = rt.zeros((77,))
    assert np.all(z.numpy() == 0)
    m = synth.normal((300, 257), 1)
    dm = rt.array(m)
    rt.causal_mask(dm, 300, 257)
    assert np.array_equal(dm.numpy(), orc.causal_mask(m))


# ---------------------------------------------------- runtime: pool, streams
def test_pool_reuses_exact_sizes(rt):
    a = rt.empty((1234,))
    p = a.ptr
    a.recycle()
    assert rt.pool_count(1234) >= 1
    b = rt.empty((1234,))
    assert b.ptr == p
    rt.reserve(4321, 3)
    assert rt.pool_count(4321) == 3


def test_streams_fork_join(rt):
    """Three forked streams compute independent GEMMs; the joined primary
    stream then consumes all three results (QkvProjection::project order)."""
    say("streams fork/join")
    streams = rt.streams_create(3)
    A = synth.uniform((256, 512), 1)
    Ws = [synth.uniform((512, 256), 10 + i) for i in range(3)]
    dA = rt.array(A)
    dWs = [rt.array(w) for w in Ws]
    outs = [rt.empty((256, 256)) for _ in range(3)]
    for _ in range(3):
        rt.streams_fork(streams)
        for s, w, o in zip(streams, dWs, outs):
            rt.gemm(dA, w, o, 256, 256, 512, stream=s)
        rt.streams_join(streams)
        total = rt.empty((256, 256))
        rt.binary(outs[0], outs[1], total, oxforge.ADD)
        rt.binary_assign(total, outs[2], oxforge.ADD)
        got = total.numpy()
        ref = [orc.gemm_f64(A, w) for w in Ws]
        assert np.max(np.abs(got - (ref[0] + ref[1] + ref[2]))) <= 1e-3


# ------------------------------------------------ executor support kernels
def test_fill_random_bit_exact(rt):
    say("fill_random")
    d = rt.empty((100_003,))
    rt.fill_random(d, 0xC0FFEE)
    assert np.array_equal(d.numpy(), orc.fill_random(100_003, 0xC0FFEE))


@pytest.mark.parametrize("act,dop", [(1, orc.MAP_GELU_D), (2, orc.MAP_RELU_D), (3, orc.MAP_SILU_D),
                                     (0, orc.MAP_IDENTITY)])
def test_activation_backward(rt, act, dop):
    say(f"activation_backward act={act}")
    dy = synth.normal((1001,), 1)
    z = synth.normal((1001,), 2, 0.0, 2.0)
    g = rt.empty((1001,))
    rt.activation_backward(rt.array(dy), rt.array(z), g, act)
    if act == 0:
        assert np.array_equal(g.numpy(), dy)
    else:
        ref = orc.activation_backward(dy, z, dop)
        assert np.all(np.abs(g.numpy() - ref) <= 2e-6 + 2e-6 * np.abs(ref))


def test_compare_counts_every_mismatch(rt):
    say("compare")
    a = synth.normal((300_000,), 1)
    b = a.copy()
    b[[0, 1023, 1024, 299_999]] += 1.0
    out = rt.empty((1,))
    rt.compare(rt.array(a), rt.array(b), out)
    assert out.numpy()[0] == 4.0
    rt.compare(rt.array(a), rt.array(a), out)
    assert out.numpy()[0] == 0.0


def test_softmax_bwd_scaled_equals_bwd_then_scale(rt):
    say("softmax_bwd_scaled")
    p = orc.softmax_rows(synth.normal((64, 300), 1))
    g = synth.normal((64, 300), 2)
    s = np.float32(1.0 / np.sqrt(np.float32(1024)))
    dp, dg = rt.array(p), rt.array(g)
    a, b = rt.empty((64, 300)), rt.empty((64, 300))
    rt.softmax_rows_bwd_scaled(dp, dg, a, 64, 300, float(s))
    rt.softmax_rows_bwd(dp, dg, b, 64, 300)
    rt.map(b, oxforge.MAP_SCALE, float(s))
    assert np.array_equal(a.numpy(), b.numpy())


@pytest.mark.parametrize("tile,splits,M,N,K", [("64x128x32_x", 2, 256, 256, 512),
                                               ("128x128x32_x", 4, 256, 256, 1024),
                                               ("128x64x32_x", 3, 128, 128, 192),
                                               ("128x128x32_x", 8, 128, 128, 256),
                                               ("64x64x32_x", 5, 128, 64, 320),
                                               ("128x64x32_x", 1, 128, 64, 64),
                                               ("64x128x32_x8", 3, 128, 256, 288)])
def test_gemm_split_k_vs_oracle(rt, tile, splits, M, N, K):
    """K slices summed in slice order: the same bar as any GEMM; one slice is
    the plain product bit for bit."""
    say(f"gemm split-K {tile} splits={splits} {M}x{N}x{K}")
    A, B = synth.uniform((M, K), 5), synth.uniform((K, N), 6)
    dA, dB, dC = rt.array(A), rt.array(B), rt.empty((M, N))
    rt.gemm_split(tile, splits, dA, dB, dC, M, N, K)
    C = dC.numpy()
    ref = orc.gemm_f64(A, B)
    absprod = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    rel_max, comp = gemm_errors(C, ref, absprod)
    assert rel_max <= 1e-4 and comp <= 1e-4, (rel_max, comp)
    if splits == 1:
        plain = rt.empty((M, N))
        rt.gemm(dA, dB, plain, M, N, K)
        assert np.array_equal(C, plain.numpy())
    with pytest.raises(oxforge.ForgeError):
        rt.gemm_split(tile, splits, dA, dB, dC, M, N, K + 16 * splits + 8)


TILES = ["128x128x32_x", "128x64x32_x", "64x128x32_x", "64x64x32_x", "64x128x32_x8",
         "64x64x16_2x2_g"]


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_every_tile_instance(rt, tile, ta, tb):
    """Each fused-epilogue instance the dispatcher can pick, at a shape that
    is two tiles by two and six K slabs: the product within the GEMM bar of
    the f64 oracle, and the
    epilogue (bias, residual, GELU, pre-activation store) bit-identical to
    the same steps applied to the plain product."""
    bm, bn = (int(x) for x in tile.split("x")[:2])
    M, N, K = 2 * bm, 2 * bn, 192
    say(f"gemm tile {tile} ta={ta} tb={tb} {M}x{N}x{K}")
    A = synth.uniform((K, M) if ta else (M, K), 31)
    B = synth.uniform((N, K) if tb else (K, N), 32)
    bias, res = synth.uniform((N,), 33), synth.uniform((M, N), 34)
    dA, dB, dbias, dres = rt.array(A), rt.array(B), rt.array(bias), rt.array(res)
    dZ, dY, dpre = rt.empty((M, N)), rt.empty((M, N)), rt.empty((M, N))
    rt.gemm_ex_tile(tile, dA, dB, dZ, M, N, K, trans_a=ta, trans_b=tb)
    Z = dZ.numpy()
    ref = orc.gemm_f64(A, B, ta, tb)
    absprod = np.abs(op_a(A, ta)).astype(np.float64) @ np.abs(op_a(B, tb)).astype(np.float64)
    rel_max, comp = gemm_errors(Z, ref, absprod)
    assert rel_max <= 1e-4 and comp <= 1e-4, (rel_max, comp)
    rt.gemm_ex_tile(tile, dA, dB, dY, M, N, K, trans_a=ta, trans_b=tb, bias=dbias, residual=dres,
                    activation=oxforge.ACT_GELU, pre_out=dpre)
    pre = (Z + bias[None, :]) + res
    assert np.array_equal(dpre.numpy(), pre)
    expect = rt.array(pre)
    rt.map(expect, oxforge.MAP_GELU, 0.0)
    assert np.array_equal(dY.numpy(), expect.numpy())
    if "_x" in tile:  # unguarded tiles refuse shapes they do not divide
        with pytest.raises(oxforge.ForgeError):
            rt.gemm_ex_tile(tile, dA, dB, dZ, M - 1, N, K, trans_a=ta, trans_b=tb)


@pytest.mark.parametrize("tile", TILES + [None])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_epilogue_row_subtrahend(rt, tile, ta, tb):
    """forge_gemm_epilogue row_sub (the softmax backward formed in the dP
    product: alpha = s, row_sub = s D, aux_mul = P): Y = ((alpha Z - r_row)
    + bias + residual) * aux bit for bit the same f32 steps applied to the
    plain product Z, on every tile instance, and through the dispatcher at a
    split-K shape (256x128x2048, the reduction kernel's epilogue) and a
    guarded one (50x70x33)."""
    shapes = [(256, 128, 2048), (50, 70, 33)] if tile is None else \
        [tuple(2 * int(x) for x in tile.split("x")[:2]) + (192,)]
    run = (lambda *a, **k: rt.gemm_ex(*a, **k)) if tile is None else \
        (lambda *a, **k: rt.gemm_ex_tile(tile, *a, **k))
    for M, N, K in shapes:
        say(f"gemm row_sub tile={tile} ta={ta} tb={tb} {M}x{N}x{K}")
        A = synth.uniform((K, M) if ta else (M, K), 41)
        B = synth.uniform((N, K) if tb else (K, N), 42)
        r, bias = synth.uniform((M,), 43), synth.uniform((N,), 44)
        res, aux = synth.uniform((M, N), 45), synth.uniform((M, N), 46)
        dA, dB, dr, dbias, dres, daux = (rt.array(v) for v in (A, B, r, bias, res, aux))
        dZ, dY, dY2 = rt.empty((M, N)), rt.empty((M, N)), rt.empty((M, N))
        run(dA, dB, dZ, M, N, K, trans_a=ta, trans_b=tb)
        Z = dZ.numpy()
        alpha = np.float32(1.0 / np.sqrt(64.0) + 0.01)
        run(dA, dB, dY, M, N, K, trans_a=ta, trans_b=tb, alpha=float(alpha), row_sub=dr,
            aux_mul=daux)
        assert np.array_equal(dY.numpy(), (alpha * Z - r[:, None]) * aux)
        run(dA, dB, dY2, M, N, K, trans_a=ta, trans_b=tb, alpha=float(alpha), row_sub=dr,
            bias=dbias, residual=dres, aux_mul=daux)
        assert np.array_equal(dY2.numpy(), (((alpha * Z - r[:, None]) + bias) + res) * aux)
    with pytest.raises(oxforge.ForgeError):  # row_sub shorter than M
        run(dA, dB, dY, M, N, K, trans_a=ta, trans_b=tb, row_sub=rt.empty((M - 1,)))


def _concat_k(mats, trans):
    """op(X_z) [rows, K] side by side along K, in the stored layout: stored
    [rows, K] concatenates columns, stored transposed [K, rows] stacks."""
    return np.ascontiguousarray(np.concatenate(mats, axis=0 if trans else 1))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("count", [2, 3])
def test_gemm_sum_equals_product_of_concatenation(rt, ta, tb, count):
    """forge_gemm_sum_f32: C = epilogue(sum_z op(A_z) op(B_z)) equals
    forge_gemm_ex_f32 on the operands concatenated along K bit for bit: on
    the one-launch K-segment path (256x128, K = 192 per product; bias,
    residual, GELU and pre-activation store; the SGD update form), and on
    the concatenating path (a guarded 50x70x33 shape, a 64x128x4096 shape the
    dispatcher splits in K, and an epilogue with column sums).  The GEMM bar
    of the f64 sum holds too."""
    shapes = [(256, 128, 192, "fused"), (256, 128, 192, "update"), (50, 70, 33, "fused"),
              (64, 128, 4096, "plain"), (256, 128, 192, "colsums")]
    for M, N, K, mode in shapes:
        say(f"gemm_sum count={count} ta={ta} tb={tb} {M}x{N}x{K} {mode}")
        As = [synth.uniform((K, M) if ta else (M, K), 400 + z) for z in range(count)]
        Bs = [synth.uniform((N, K) if tb else (K, N), 410 + z) for z in range(count)]
        bias, res = synth.uniform((N,), 420), synth.uniform((M, N), 421)
        W0 = synth.uniform((M, N), 422)
        dA, dB = [rt.array(a) for a in As], [rt.array(b) for b in Bs]
        dAc, dBc = rt.array(_concat_k(As, ta)), rt.array(_concat_k(Bs, not tb))
        kw = {}
        if mode == "fused":
            kw = dict(bias=rt.array(bias), residual=rt.array(res),
                      activation=oxforge.ACT_GELU)
        outs = []
        for run in ("sum", "concat"):
            C = rt.array(W0) if mode == "update" else rt.empty((M, N))
            pre = rt.empty((M, N)) if mode == "fused" else None
            ex = dict(kw)
            if pre is not None:
                ex["pre_out"] = pre
            if mode == "update":
                ex.update(update=True, update_scale=1e-3)
            cs = rt.empty((N,)) if mode == "colsums" else None
            if cs is not None:
                ex["col_sums_out"] = cs
            if run == "sum":
                rt.gemm_sum(dA, dB, C, M, N, K, trans_a=ta, trans_b=tb, **ex)
            else:
                rt.gemm_ex(dAc, dBc, C, M, N, count * K, trans_a=ta, trans_b=tb, **ex)
            outs.append([C.numpy()] + ([pre.numpy()] if pre is not None else []) +
                        ([cs.numpy()] if cs is not None else []))
        for a, b in zip(outs[0], outs[1]):
            assert np.array_equal(a, b), mode
        if mode == "plain":
            ref = sum(orc.gemm_f64(a, b, ta, tb) for a, b in zip(As, Bs))
            assert np.max(np.abs(outs[0][0] - ref)) / np.max(np.abs(ref)) <= 1e-4
    with pytest.raises(oxforge.ForgeError):  # four products
        rt.gemm_sum(dA + dA[:4 - count], dB + dB[:4 - count], C, M, N, K, trans_a=ta,
                    trans_b=tb)
    # one product is the fused product itself; K = 0 gives the epilogue of zeros
    C1, C2 = rt.empty((M, N)), rt.empty((M, N))
    rt.gemm_sum(dA[:1], dB[:1], C1, M, N, K, trans_a=ta, trans_b=tb, bias=rt.array(bias))
    rt.gemm_ex(dA[0], dB[0], C2, M, N, K, trans_a=ta, trans_b=tb, bias=rt.array(bias))
    assert np.array_equal(C1.numpy(), C2.numpy())
    empty = [rt.empty((0,)) for _ in range(count)]
    rt.gemm_sum(empty, empty, C1, M, N, 0, trans_a=ta, trans_b=tb, bias=rt.array(bias))
    assert np.array_equal(C1.numpy(), np.broadcast_to(bias, (M, N)))


U32 = 2.0 ** -24


def _rms_rows(Y, eps=1e-5):
    Y = np.asarray(Y, np.float64)
    return np.sqrt((Y * Y).mean(axis=1, keepdims=True) + eps)


def _check_row_sumsq(sq, Y):
    """sq [M, ceil(N/32)] against the f64 sums of squares of the stored Y
    over each 32-column block: at most 40 u times the sum (each block sum
    passes a term through at most 35 roundings: its square, 31 adds)."""
    Y = np.asarray(Y, np.float64)
    M, N = Y.shape
    P = -(-N // 32)
    pad = np.zeros((M, P * 32))
    pad[:, :N] = Y * Y
    ref = pad.reshape(M, P, 32).sum(axis=2)
    assert sq.shape == (M * P,)
    assert np.all(np.abs(sq.reshape(M, P) - ref) <= 40 * U32 * ref + 1e-30)


def _check_col_sums(sums, Y):
    """Column sums of the stored Y: within M u times the column's sum of
    magnitudes (first-order bound for any order of at most M - 1 adds per
    term, plus the final pass)."""
    Y = np.asarray(Y, np.float64)
    M = Y.shape[0]
    ref = Y.sum(axis=0)
    assert np.all(np.abs(sums - ref) <= (M + 16) * U32 * np.abs(Y).sum(axis=0))


STAT_TILES = TILES + [None]


@pytest.mark.parametrize("tile", STAT_TILES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("N", [384, 192, 352])
def test_gemm_epilogue_row_statistics_and_column_sums(rt, tile, ta, tb, N):
    """The epilogue's row statistics and column sums (forge_gemm_epilogue
    row_parts_in / row_div / row_sumsq_out / col_sums_*) on every tile
    instance and through the dispatcher (None): a parameterless RMSNorm of
    the first product's rows folded into a second product, as the C4 block
    folds it across its GEMM boundaries (norm.rs:50-69 with
    inference.rs:90-108):
      Y1 = op(A) op(B) + R, with the sums of squares of Y1's 32-column blocks;
      Z  = (Y1 / d) W + b, d_r = sqrt(mean_c Y1[r, c]^2 + eps), divisor
           formed from those sums (row_div bit 0);
      Z2 = Y1 W2 + b2 + Y1 / d (bit 1, the residual divided);
    and the column sums of Z with a parameter's SGD step.  Products within
    the GEMM bar (1e-4 of the f64 result on the GPU's own Y1); sums within
    their rounding bounds; the parameter step bit for bit against the
    returned sums.  N = 192 gives 6 partials per row (the unguarded tiles'
    scalar row-scale loads), N = 352 shapes no unguarded tile divides."""
    M, K = 256, 160
    bn = 64 if tile is None else int(tile.split("x")[1])
    if tile is not None and N % bn:
        pytest.skip("the tile does not divide N")
    say(f"gemm row statistics tile={tile} ta={ta} tb={tb} N={N}")
    run = (lambda *a, **k: rt.gemm_ex(*a, **k)) if tile is None else \
        (lambda *a, **k: rt.gemm_ex_tile(tile, *a, **k))
    A = synth.uniform((K, M) if ta else (M, K), 81)
    B = synth.uniform((N, K) if tb else (K, N), 82)
    R = synth.uniform((M, N), 83)
    W = synth.uniform((N, N), 84)
    b = synth.uniform((N,), 85)
    dA, dB, dR, dW, db = (rt.array(v) for v in (A, B, R, W, b))
    P = -(-N // 32)
    dY1, sq = rt.empty((M, N)), rt.empty((M * P,))
    run(dA, dB, dY1, M, N, K, trans_a=ta, trans_b=tb, residual=dR, row_sumsq_out=sq)
    Y1 = dY1.numpy()
    ref1 = orc.gemm_f64(A, B, ta, tb) + R
    assert np.max(np.abs(Y1 - ref1)) / np.max(np.abs(ref1)) <= 1e-4
    _check_row_sumsq(sq.numpy(), Y1)

    h = Y1.astype(np.float64) / _rms_rows(Y1)
    dZ, cs, par = rt.empty((M, N)), rt.empty((N,)), rt.array(b)
    run(dY1, dW, dZ, M, N, N, bias=db, row_parts_in=sq, row_parts=P, row_n=N, row_eps=1e-5,
        row_div=1, col_sums_out=cs, col_sums_param=par, col_sums_lr=1e-3)
    Z = dZ.numpy()
    refz = h @ W.astype(np.float64) + b
    assert np.max(np.abs(Z - refz)) / np.max(np.abs(refz)) <= 1e-4
    sums = cs.numpy()
    _check_col_sums(sums, Z)
    assert np.array_equal(par.numpy(), b - np.float32(1e-3) * sums)

    dZ2 = rt.empty((M, N))
    run(dY1, dW, dZ2, M, N, N, bias=db, residual=dY1, row_parts_in=sq, row_parts=P, row_n=N,
        row_eps=1e-5, row_div=2)
    refz2 = Y1.astype(np.float64) @ W.astype(np.float64) + b + h
    Z2 = dZ2.numpy()
    assert np.max(np.abs(Z2 - refz2)) / np.max(np.abs(refz2)) <= 1e-4


def test_gemm_epilogue_statistics_on_split_and_guarded_products(rt):
    """The same statistics where the dispatcher splits K (a 64 x 128 output
    over K = 4096) or takes the bounds-guarded tile (odd sizes): the
    divisors, sums of squares and column sums then come from separate
    passes over C, with the same results to within rounding; column sums
    of no rows are zero and leave the parameter."""
    for M, N, K in ((64, 128, 4096), (70, 50, 33)):
        name = rt.gemm_kernel_name(M, N, K, fused=True)
        say(f"gemm statistics {M}x{N}x{K} via {name}")
        assert ("split" in name) == (K == 4096) and ("2x2_g" in name) == (K == 33)
        A, B = synth.uniform((M, K), 91), synth.uniform((K, N), 92)
        W = synth.uniform((N, N), 93)
        P = -(-N // 32)
        dA, dB, dW = rt.array(A), rt.array(B), rt.array(W)
        dY1, sq = rt.empty((M, N)), rt.empty((M * P,))
        rt.gemm_ex(dA, dB, dY1, M, N, K, row_sumsq_out=sq)
        Y1 = dY1.numpy()
        _check_row_sumsq(sq.numpy(), Y1)
        dZ, cs = rt.empty((M, N)), rt.empty((N,))
        rt.gemm_ex(dY1, dW, dZ, M, N, N, row_parts_in=sq, row_parts=P, row_n=N, row_eps=1e-5,
                   row_div=1, col_sums_out=cs)
        Z = dZ.numpy()
        refz = Y1.astype(np.float64) / _rms_rows(Y1) @ W.astype(np.float64)
        assert np.max(np.abs(Z - refz)) / np.max(np.abs(refz)) <= 1e-4
        _check_col_sums(cs.numpy(), Z)
    cs = rt.array(np.full(8, 3.0, np.float32))
    par = rt.array(np.full(8, 2.0, np.float32))
    empty = rt.empty((0,))
    rt.gemm_ex(empty, rt.empty((4 * 8,)), empty, 0, 8, 4, col_sums_out=cs, col_sums_param=par,
               col_sums_lr=0.5)
    assert np.all(cs.numpy() == 0) and np.all(par.numpy() == 2.0)
    with pytest.raises(oxforge.ForgeError):  # row_div without row statistics
        rt.gemm_ex(dA, dB, dY1, 64, 128, 4096, row_div=1)


@pytest.mark.parametrize("M,N,K,ta,tb,fused", [(4096, 4096, 4096, 0, 0, 0),
                                                (2048, 2048, 1024, 0, 1, 1),
                                                (4096, 1024, 2048, 0, 0, 0),
                                                (2048, 1024, 4096, 0, 0, 1),
                                                (4096, 2048, 2048, 1, 0, 1),
                                                (256, 256, 512, 1, 1, 1),
                                                (96, 80, 40, 0, 0, 0)])
def test_gemm_kernel_name_names_the_kernel_that_runs(rt, M, N, K, ta, tb, fused):
    """forge_gemm_kernel_name reports the dispatcher's choice: the product
    through that tile instance equals the dispatched product bit for bit."""
    name = rt.gemm_kernel_name(M, N, K, ta, tb, fused)
    say(f"gemm kernel name {M}x{N}x{K} ta={ta} tb={tb} fused={fused}: {name}")
    ab = ("t" if ta else "n") + ("t" if tb else "n")
    prefix = f"forge_gemm_{ab}_"
    assert name.startswith(prefix) and "/split" not in name, name
    kernel, _, cap = name.partition("@")
    plain = not fused and ab == "nn"
    assert kernel.endswith("_e") != plain, name
    tag = kernel[len(prefix):].removesuffix("_e") + (f"@{cap}" if cap else "")
    A = synth.uniform((K, M) if ta else (M, K), 41)
    B = synth.uniform((N, K) if tb else (K, N), 42)
    dA, dB, dC, dT = rt.array(A), rt.array(B), rt.empty((M, N)), rt.empty((M, N))
    if plain:
        rt.gemm(dA, dB, dC, M, N, K)
        rt.gemm_tile(tag, dA, dB, dT, M, N, K)
    else:
        rt.gemm_ex(dA, dB, dC, M, N, K, trans_a=ta, trans_b=tb)
        rt.gemm_ex_tile(tag, dA, dB, dT, M, N, K, trans_a=ta, trans_b=tb)
    assert np.array_equal(dC.numpy(), dT.numpy())


@pytest.mark.parametrize("tile", ["64x128x32_x@2", "128x128x32_x@1", "64x64x32_x@3",
                                  "128x64x32_x@2", "64x128x32_x8@1"])
def test_gemm_occupancy_cap_keeps_results(rt, tile):
    """A launch that lets a CU hold fewer workgroups computes the same
    product bit for bit, plain and with a fused epilogue; malformed caps are
    refused."""
    M, N, K = 512, 512, 256
    say(f"gemm occupancy cap {tile}")
    base = tile.partition("@")[0]
    A, B, bias = synth.uniform((M, K), 51), synth.uniform((K, N), 52), synth.uniform((N,), 53)
    dA, dB, dbias = rt.array(A), rt.array(B), rt.array(bias)
    out = [rt.empty((M, N)) for _ in range(4)]
    rt.gemm_tile(base, dA, dB, out[0], M, N, K)
    rt.gemm_tile(tile, dA, dB, out[1], M, N, K)
    rt.gemm_ex_tile(base, dA, dB, out[2], M, N, K, bias=dbias, activation=oxforge.ACT_GELU)
    rt.gemm_ex_tile(tile, dA, dB, out[3], M, N, K, bias=dbias, activation=oxforge.ACT_GELU)
    assert np.array_equal(out[0].numpy(), out[1].numpy())
    assert np.array_equal(out[2].numpy(), out[3].numpy())
    for bad in (base + "@0", base + "@17", base + "@x"):
        with pytest.raises(oxforge.ForgeError):
            rt.gemm_tile(bad, dA, dB, out[1], M, N, K)


@pytest.mark.parametrize("M,N,K", [(256, 128, 192), (70, 50, 33)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_batch_bit_identical_to_single(rt, M, N, K, ta, tb):
    """Three products with different fused epilogues in one launch equal
    three forge_gemm_ex_f32 calls bit for bit."""
    say(f"gemm batch {M}x{N}x{K} ta={ta} tb={tb}")
    rng = np.random.default_rng(M + 2 * ta + tb)

    def mat(*shape):
        return rng.uniform(-1, 1, shape).astype(np.float32)

    As = [rt.array(mat(*((K, M) if ta else (M, K)))) for _ in range(3)]
    Bs = [rt.array(mat(*((N, K) if tb else (K, N)))) for _ in range(3)]
    bias, res, c0 = rt.array(mat(N)), rt.array(mat(M, N)), mat(M, N)
    eps = [dict(bias=None, activation=oxforge.ACT_GELU),
           dict(alpha=0.125, residual=res),
           dict(update=True, update_scale=0.01)]
    eps[0]["bias"] = bias
    outs = {}
    for mode in ("batch", "single"):
        Cs = [rt.array(c0) for _ in range(3)]
        pres = [rt.empty((M, N)) for _ in range(3)]
        problems = []
        for z in range(3):
            ep = dict(eps[z], pre_out=pres[z])
            problems.append((As[z], Bs[z], Cs[z], ep))
        if mode == "batch":
            rt.gemm_batch(problems, M, N, K, trans_a=bool(ta), trans_b=bool(tb))
        else:
            for A, B, C, ep in problems:
                rt.gemm_ex(A, B, C, M, N, K, trans_a=bool(ta), trans_b=bool(tb), **ep)
        outs[mode] = [c.numpy() for c in Cs] + [p.numpy() for p in pres]
    for a, b in zip(outs["batch"], outs["single"]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("n", [1, 7, 1024, 100_003])
def test_sgd_update_bit_exact(rt, n):
    """param - lr * grad with two roundings, as the reference's clone / scale /
    subtract sequence (linear.rs:385-390)."""
    say(f"sgd_update n={n}")
    p, g = synth.normal((n,), 1), synth.normal((n,), 2)
    lr = np.float32(3e-3)
    dp = rt.array(p)
    rt.sgd_update(dp, rt.array(g), float(lr))
    assert np.array_equal(dp.numpy(), p - lr * g)
    # Unaligned views take the scalar kernel.
    dp2 = rt.array(np.concatenate([[0.0], p]).astype(np.float32)).view(1, (n,))
    dg2 = rt.array(np.concatenate([[0.0], g]).astype(np.float32)).view(1, (n,))
    rt.sgd_update(dp2, dg2, float(lr))
    assert np.array_equal(dp2.numpy(), p - lr * g)


@pytest.mark.parametrize("rows,cols", [(64, 1024), (33, 70)])
def test_norm_out_of_place_equals_in_place(rt, rows, cols):
    say(f"norm out-of-place {rows}x{cols}")
    x = synth.normal((rows, cols), 3)
    gm, bt = synth.normal((cols,), 4, 1.0, 0.1), synth.normal((cols,), 5, 0.0, 0.1)
    dgm, dbt = rt.array(gm), rt.array(bt)
    for name, args in (("layer", (dgm, dbt)), ("rms", (dgm,))):
        src, inplace, out = rt.array(x), rt.array(x), rt.empty((rows, cols))
        getattr(rt, f"{name}_norm")(inplace, rows, cols, *args)
        getattr(rt, f"{name}_norm_out")(src, out, rows, cols, *args)
        assert np.array_equal(out.numpy(), inplace.numpy()), name
        assert np.array_equal(src.numpy(), x), f"{name}: input modified"
    # Partial overlap of input and output is rejected.
    big = rt.array(np.zeros((rows + 1) * cols, np.float32))
    with pytest.raises(oxforge.ForgeError):
        rt.layer_norm_out(big.view(0, (rows, cols)), big.view(cols, (rows, cols)), rows, cols)


@pytest.mark.parametrize("M,N,K", [(256, 128, 192), (70, 50, 33)])
def test_transposed_operands_bit_identical_to_materialised_transpose(rt, M, N, K):
    """NT/TN GEMMs read A^T/B^T in place; the products equal the reference's
    transpose-then-GEMM sequence bit for bit."""
    say(f"nt/tn vs transpose {M}x{N}x{K}")
    At = synth.uniform((K, M), 1)
    Bt = synth.uniform((N, K), 2)
    B = synth.uniform((K, N), 3)
    dAt, dBt, dB = rt.array(At), rt.array(Bt), rt.array(B)
    dA, dBn = rt.empty((M, K)), rt.empty((K, N))
    rt.transpose(dAt, dA, K, M)
    rt.transpose(dBt, dBn, N, K)
    c1, c2 = rt.empty((M, N)), rt.empty((M, N))
    rt.gemm_ex(dAt, dB, c1, M, N, K, trans_a=True)
    rt.gemm_ex(dA, dB, c2, M, N, K)
    assert np.array_equal(c1.numpy(), c2.numpy())
    rt.gemm_ex(dA, dBt, c1, M, N, K, trans_b=True)
    rt.gemm_ex(dA, dBn, c2, M, N, K)
    assert np.array_equal(c1.numpy(), c2.numpy())


def test_zero_sized_inputs(rt):
    """Every entry point accepts zero-sized shapes (the reference's spans
    and matrices may be empty, span.rs:302-359) and writes only what the
    empty case defines: a sum over no elements or rows is 0, a max over
    none is f32::MIN (span.rs:319-321), and a norm backward over no rows
    gives zero dgamma / dbeta and leaves gamma / beta where its SGD step
    would move them.  Everything else is left as it was."""
    say("zero-sized inputs")
    sent = np.full(16, 7.0, np.float32)
    a, b, o = rt.array(sent), rt.array(sent), rt.array(sent)

    def untouched(*xs):
        return all(np.array_equal(x.numpy(), sent) for x in xs)

    rt.binary(a, b, o, oxforge.ADD, n=0)
    rt.binary_assign(o, a, oxforge.MUL, n=0)
    rt.map(o, oxforge.MAP_GELU, n=0)
    rt.fill_seq(o, n=0)
    rt.fill_random(o, 5, n=0)
    rt.sgd_update(o, a, 0.1, n=0)
    rt.activation_backward(a, b, o, oxforge.ACT_GELU, n=0)
    rt.copy(o, a, n=0)
    for M, N, K in ((0, 4, 4), (4, 0, 4)):
        rt.gemm(a, b, o, M, N, K)
    assert untouched(a, b, o)
    for rows, cols in ((0, 4), (4, 0)):
        rt.softmax_rows(o, rows, cols)
        rt.layer_norm(o, rows, cols, a, b)
        rt.rms_norm(o, rows, cols, a)
        rt.softmax_rows_bwd(a, b, o, rows, cols)
        rt.binary_assign_by_rows(o, a, rows, cols, oxforge.ADD)
        rt.causal_mask(o, rows, cols)
        rt.transpose(a, o, rows, cols)
        rt.layer_norm_bwd(a, b, o, rows, cols)
        rt.rms_norm_bwd(a, b, o, rows, cols)
        assert untouched(a, b, o), (rows, cols)

    # Sums over empty ranges are zero; the max over none is f32::MIN.
    s = rt.array(sent)
    rt.sum_rows(a, s, 4, 0)
    assert np.array_equal(s.numpy()[:4], np.zeros(4, np.float32))
    assert np.array_equal(s.numpy()[4:], sent[4:])
    s = rt.array(sent)
    rt.sum_cols(a, s, 0, 4)
    assert np.array_equal(s.numpy()[:4], np.zeros(4, np.float32))
    assert np.array_equal(s.numpy()[4:], sent[4:])
    s = rt.array(sent)
    rt.reduce_sum(a, s, n=0)
    rt.map_sum(a, s.view(1, (1,)), oxforge.MAP_HALF_SQ, n=0)
    rt.compare(a, b, s.view(2, (1,)), n=0)
    rt.reduce_max(a, s.view(3, (1,)), n=0)
    assert np.array_equal(s.numpy()[:4], np.array([0, 0, 0, -3.4028235e38], np.float32))

    # Norm backward over no rows: zero gradients; the SGD step leaves the
    # parameters as they are.
    gam, bet, dg, db = rt.array(sent), rt.array(sent), rt.array(sent), rt.array(sent)
    rt.layer_norm_bwd(a, b, o, 0, 4, gam, dg, db)
    assert np.array_equal(dg.numpy()[:4], np.zeros(4, np.float32))
    assert np.array_equal(db.numpy()[:4], np.zeros(4, np.float32))
    dg, db = rt.array(sent), rt.array(sent)
    rt.layer_norm_bwd_sgd(a, b, o, 0, 4, 0.5, gam, bet, dg, db)
    rt.rms_norm_bwd_sgd(a, b, o, 0, 4, 0.5, gam, dg)
    assert np.array_equal(dg.numpy()[:4], np.zeros(4, np.float32))
    assert np.array_equal(db.numpy()[:4], np.zeros(4, np.float32))
    assert untouched(gam, bet, o)
    s = rt.array(sent)
    prm = rt.array(sent)
    rt.sum_cols_sgd(a, 0, 4, 0.5, out=s, param=prm)
    assert np.array_equal(s.numpy()[:4], np.zeros(4, np.float32))
    assert untouched(prm)


def hash_fill(seed, start, count):
    """forge_fill_random's values at indices start .. start + count - 1:
    common.rs:3-9 on the wrapping u32 seed + index, divided by u32::MAX as
    f32 (elementwise.rs:40-41), restated in numpy."""
    x = (np.uint64(seed) + np.arange(start, start + count, dtype=np.uint64)) & 0xFFFFFFFF
    x = (x + (x << 13)) & 0xFFFFFFFF
    x = (x - (x >> 17)) & 0xFFFFFFFF
    x = (x * ((x << 5) & 0xFFFFFFFF)) & 0xFFFFFFFF
    return x.astype(np.float32) / np.float32(4294967295.0)


def test_operands_beyond_4gib(rt):
    """Operands of 4.0018 GiB (1,074,266,112 floats), filled on the device:
    rows and elements past the 4 GiB byte offset go through the GEMM (A of
    [262272, 4096]), the row kernels ([1049088, 1024]) and the streaming
    kernels at the same bars as everywhere else, checked on sampled rows."""
    n = 262272 * 4096
    say(f"operands beyond 4 GiB: {n} floats")
    a, b, c = rt.empty((n,)), rt.empty((n,)), rt.empty((n,))
    rt.fill_random(a, 11)
    rt.fill_random(b, 12)

    # GEMM: A [262272, 4096] x B [4096, 64].
    M, K, N = 262272, 4096, 64
    B = synth.uniform((K, N), 13)
    dB, dC = rt.array(B), rt.empty((M, N))
    rt.gemm(a, dB, dC, M, N, K)
    for r in (0, 262143, 262144, 262271):  # 262144 * 4096 * 4 B = 4 GiB
        Ar = hash_fill(11, r * K, K)
        ref = Ar.astype(np.float64) @ B.astype(np.float64)
        got = dC.view(r * N, (N,)).numpy().astype(np.float64)
        absprod = np.abs(Ar).astype(np.float64) @ np.abs(B).astype(np.float64)
        assert np.max(np.abs(got - ref) / absprod) <= 1e-4, r

    # Streaming: c = a + b, bit-exact past 2^30 floats.
    rt.binary(a, b, c, oxforge.ADD)
    for start in (0, 2**30 - 8, n - 4096):
        want = hash_fill(11, start, 4096) + hash_fill(12, start, 4096)
        assert np.array_equal(c.view(start, (4096,)).numpy(), want), start

    # Row kernels on [1049088, 1024]: softmax in place, LayerNorm backward.
    rows, cols = 1049088, 1024
    rt.layer_norm_bwd(a, b, c, rows, cols)
    for r in (0, 1048575, 1048576, rows - 1):  # row 1048576 starts at 4 GiB
        x, dy = hash_fill(11, r * cols, cols)[None, :], hash_fill(12, r * cols, cols)[None, :]
        dx = c.view(r * cols, (1, cols)).numpy()
        assert np.max(np.abs(dx - orc.layer_norm_backward(x, dy, None))) <= TOL_ROW, r
    rt.softmax_rows(a, rows, cols)
    for r in (0, 1048576, rows - 1):
        x = hash_fill(11, r * cols, cols)[None, :]
        got = a.view(r * cols, (1, cols)).numpy()
        assert np.max(np.abs(got - orc.softmax_rows(x))) <= TOL_ROW, r
    for d in (a, b, c, dB, dC):
        d.recycle()


def test_gemm_pitch_beyond_unguarded_limit(rt):
    """A row pitch above 2^21 floats (A^T of [64, 2^21 + 64] in a TN
    product) goes to the bounds-guarded kernel, whose offsets are 64-bit;
    rows on both sides of the 2^21 boundary match the f64 oracle."""
    M, N, K = 2**21 + 64, 64, 64
    say(f"gemm pitch {M} (tn)")
    assert "_g" in rt.gemm_kernel_name(M, N, K, trans_a=True, fused=True)
    at = rt.empty((K, M))
    rt.fill_random(at, 21)
    B = synth.uniform((K, N), 22)
    dB, dC = rt.array(B), rt.empty((M, N))
    rt.gemm_ex(at, dB, dC, M, N, K, trans_a=True)
    for m in (0, 2**21 - 1, 2**21, M - 1):
        a_row = np.array([hash_fill(21, k * M + m, 1)[0] for k in range(K)], np.float32)
        ref = a_row.astype(np.float64) @ B.astype(np.float64)
        absprod = np.abs(a_row).astype(np.float64) @ np.abs(B).astype(np.float64)
        got = dC.view(m * N, (N,)).numpy().astype(np.float64)
        assert np.max(np.abs(got - ref) / absprod) <= 1e-4, m
    for d in (at, dB, dC):
        d.recycle()


def test_runtime_plumbing(rt):
    """Device properties, events, stream waits and destruction, forge_free
    and the causal mask on a block of query rows (the chunked-attention
    form of row.rs:5-14): results against host arithmetic or the oracle."""
    from oxforge._lib import call

    say("runtime plumbing")
    props = rt.props()
    assert props["cu_count"] > 0 and props["lds_bytes"] >= 65536
    assert props["arch"].startswith("gfx950")

    # Events bracket device work on a stream; elapsed time is positive and
    # the recorded work is complete once it is read.
    x = rt.array(np.zeros(1 << 20, np.float32))
    e0, e1 = rt.event(), rt.event()
    rt.record(e0)
    for _ in range(8):
        rt.map(x, oxforge.MAP_ADD, 1.0)
    rt.record(e1)
    assert rt.elapsed_ms(e0, e1) > 0.0
    assert np.array_equal(x.numpy(), np.full(1 << 20, 8.0, np.float32))
    rt.event_destroy(e0)
    rt.event_destroy(e1)

    # A stream waits for work queued on another; destroyed streams are gone.
    s1, s2 = rt.streams_create(2)
    y = rt.array(np.zeros(1 << 20, np.float32))
    rt.sync()  # the upload is ordered on the primary stream only
    for _ in range(4):
        rt.map(y, oxforge.MAP_ADD, 1.0, stream=s1)
    rt.stream_wait(s2, s1)
    rt.map(y, oxforge.MAP_SCALE, 2.0, stream=s2)
    rt.sync(s2)
    assert np.array_equal(y.numpy(), np.full(1 << 20, 8.0, np.float32))
    for s in (s1, s2):
        call("forge_stream_destroy", rt.handle, s)

    # forge_free releases a buffer instead of returning it to the pool.
    n = 12345
    a, b = rt.empty((n,)), rt.empty((n,))
    held = rt.pool_count(n)
    rt.free(a)
    assert rt.pool_count(n) == held
    b.recycle()
    assert rt.pool_count(n) == held + 1

    # The causal mask of query rows r0 .. r0 + rows - 1 of an [S, S] score
    # matrix equals those rows of the full mask.
    S, cols = 200, 200
    full = synth.normal((S, cols), 9)
    ref = orc.causal_mask(full)
    for r0, rows in ((0, 64), (64, 64), (128, 72), (199, 1)):
        blk = rt.array(full[r0:r0 + rows])
        call("forge_causal_mask_rows", rt.handle, None, blk.slice, rows, cols, r0)
        assert np.array_equal(blk.numpy(), ref[r0:r0 + rows]), r0
    with pytest.raises(oxforge.ForgeError):
        blk = rt.empty((2, 4))
        call("forge_causal_mask_rows", rt.handle, None, blk.slice, 2, 4, 2**31 - 2)


@pytest.mark.parametrize("cols", [64, 1000, 4096, 5000])
def test_row_kernels_special_values(rt, cols):
    """Rows holding NaN, +inf, -inf or one constant value: the GPU's NaN and
    infinity positions equal the oracle's (the reference's arithmetic: a
    NaN or +inf poisons a softmax or LayerNorm row, -inf only zeroes its
    softmax entry, a constant row normalises to zeros), and finite entries
    meet the usual bar."""
    say(f"row special values cols={cols}")
    x = synth.normal((6, cols), 31)
    x[0, 5] = np.nan
    x[1, :] = 3.0
    x[2, 7] = np.inf
    x[3, 9] = -np.inf
    x[4, 1] = np.inf
    x[4, 2] = -np.inf
    for name, fn, ref in (("softmax", lambda d: rt.softmax_rows(d, 6, cols), orc.softmax_rows(x)),
                          ("layer_norm", lambda d: rt.layer_norm(d, 6, cols), orc.layer_norm(x)),
                          ("rms_norm", lambda d: rt.rms_norm(d, 6, cols), orc.rms_norm(x))):
        d = rt.array(x)
        fn(d)
        got = d.numpy()
        assert np.array_equal(np.isnan(got), np.isnan(ref)), name
        assert np.array_equal(np.isinf(got), np.isinf(ref)), name
        fin = np.isfinite(ref)
        assert np.max(np.abs(got[fin] - ref[fin]), initial=0.0) <= TOL_ROW, name
