"""Kernel-level parity of the HIP path (through the C-ABI) against the CPU
oracle on the same seeded inputs.

Tolerances: fp32 paths 1e-4 max-abs; bf16 / fp8 paths 2e-2
relative (per row ||d||_inf / ||ref||_inf); integer / byte work bit-exact.
"""
import ctypes

import numpy as np
import pytest

from helpers import bf16_dev, bits_u16, ptr, row_rel_err, rng, stream, sync, to_dev

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
LOWP_TOL = 2e-2


def _gemm(cbis, M, N, K, X, x_dtype, W, w_dtype, Y, y_dtype, bias=None, w_scale=None, gelu=False, residual=None,
          kv=None, workspace=False):
    d = cbis.GemmDesc()
    d.M, d.N, d.K = M, N, K
    d.x_dtype, d.X, d.ldx = x_dtype, ptr(X), K
    d.w_dtype, d.W, d.ldw = w_dtype, ptr(W), K
    d.w_scale = ptr(w_scale)
    d.bias = ptr(bias)
    d.epilogue = cbis.EPI_GELU if gelu else cbis.EPI_NONE
    d.residual, d.ldr = ptr(residual), N
    d.y_dtype, d.Y, d.ldy = y_dtype, ptr(Y), (kv["ldy"] if kv else N)
    if kv:
        d.kv_col0, d.kv_width, d.kv_dtype, d.page_size = kv["col0"], kv["width"], kv["dtype"], 16
        d.k_pool, d.v_pool = ptr(kv["k"]), ptr(kv["v"])
        d.write_page, d.write_offset = ptr(kv["wpage"]), ptr(kv["woff"])
    ws = None
    if workspace:
        import torch
        need = cbis.kernels().cbis_gemm_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=Y.device)
        d.workspace, d.workspace_bytes = ptr(ws), need
    cbis.check(cbis.kernels().cbis_gemm(ctypes.byref(d), stream()), "cbis_gemm")
    sync()
    return d.workspace_bytes


# --------------------------------------------------------------------------
# synthetic data and number formats: bit-exact
# --------------------------------------------------------------------------

def test_fill_normal_exact_matches_oracle_prng(cbis, oracle, dev):
    import torch
    n = 200_003
    out = torch.empty(n, dtype=torch.float32, device=dev)
    cbis.check(cbis.kernels().cbis_fill_normal_exact(ptr(out), cbis.F32, n, 0, 105, 777, 0.02, stream()))
    sync()
    ref = oracle.normal(0, 105, n, 0.02, start=777)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    outb = torch.empty(n, dtype=torch.bfloat16, device=dev)
    cbis.check(cbis.kernels().cbis_fill_normal_exact(ptr(outb), cbis.BF16, n, 3, 2, 0, 1.0, stream()))
    sync()
    assert np.array_equal(bits_u16(outb), oracle.f32_to_bf16_bits(oracle.normal(3, 2, n, 1.0)))


def test_convert_bf16_and_fp8_quantise_bit_exact(cbis, oracle, dev):
    import torch
    g = rng(1)
    N, K = 96, 512
    w = (g.standard_normal((N, K)) * 0.02).astype(np.float32)
    # exact rounding ties and extremes for both codecs
    w[0, :8] = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 0.0, -0.0, 1e-30, 3e38, -3e38], np.float32)
    w[1, :4] = np.array([448.0, -448.0, 300.0, 2 ** -10], np.float32) * 1e-3
    w[2, :] = 0.0  # all-zero row: scale 1
    src = to_dev(w, dev)
    b = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    cbis.check(cbis.kernels().cbis_convert_f32(ptr(b), cbis.BF16, ptr(src), N * K, stream()))
    codes = torch.empty((N, K), dtype=torch.uint8, device=dev)
    scale = torch.empty(N, dtype=torch.float32, device=dev)
    cbis.check(cbis.kernels().cbis_quantize_fp8_rows(ptr(codes), ptr(scale), ptr(src), N, K, stream()))
    sync()
    assert np.array_equal(bits_u16(b), oracle.f32_to_bf16_bits(w))
    ref_codes, ref_scale = oracle.quantize_e4m3_rows(w)
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), ref_scale.view(np.uint32))
    assert np.array_equal(codes.cpu().numpy(), ref_codes)


# --------------------------------------------------------------------------
# GEMM
# --------------------------------------------------------------------------

C2_SHAPES = [  # (name, N, K, bias, gelu, residual): config 2
    ("qkv", 768, 256, True, False, False),
    ("out", 256, 256, True, False, False),
    ("up", 1024, 256, True, True, False),
    ("down", 256, 1024, True, False, True),
]


def _sample_rows(M, k, seed):
    if M <= k:
        return np.arange(M)
    r = rng(seed).choice(M, size=k, replace=False)
    r.sort()
    return r


@pytest.mark.parametrize("ws", [False, True], ids=["no_ws", "split_ws"])
@pytest.mark.parametrize("M", [64, 512, 4096])
@pytest.mark.parametrize("shape", C2_SHAPES, ids=lambda s: s[0])
def test_gemm_fp32_c2(cbis, oracle, dev, M, shape, ws):
    """fp32 C2 shapes; with the workspace cbis_gemm_workspace_size asks for,
    the grids too small to fill the CUs split K (M = 512 all four shapes,
    M = 4096 MLP down) and the partials are reduced with the epilogue."""
    import torch
    name, N, K, has_b, gelu, has_r = shape
    x = oracle.normal(11, 1, M * K).reshape(M, K)
    w = oracle.normal(11, 2, N * K, 0.02).reshape(N, K)
    b = oracle.normal(11, 3, N, 0.02) if has_b else None
    r = oracle.normal(11, 4, M * N).reshape(M, N) if has_r else None
    X, W = to_dev(x, dev), to_dev(w, dev)
    B = to_dev(b, dev) if has_b else None
    Y = to_dev(r, dev) if has_r else torch.empty((M, N), dtype=torch.float32, device=dev)
    used = _gemm(cbis, M, N, K, X, cbis.F32, W, cbis.F32, Y, cbis.F32, bias=B, gelu=gelu,
                 residual=Y if has_r else None, workspace=ws)
    if ws:
        assert (used > 0) == (M == 512 or (M == 4096 and name == "down")), used
    rows = _sample_rows(M, 512, M)
    ref = oracle.gemm(x[rows], w, bias=b, gelu=gelu, residual=None if r is None else r[rows])
    err = np.abs(Y.cpu().numpy()[rows] - ref).max()
    assert err < FP32_TOL, err


@pytest.mark.parametrize("M", [64, 512, 4096])
@pytest.mark.parametrize("shape", C2_SHAPES, ids=lambda s: s[0])
def test_gemm_bf16_c2(cbis, oracle, dev, M, shape):
    import torch
    name, N, K, has_b, gelu, has_r = shape
    X, x = bf16_dev(oracle.normal(12, 1, M * K).reshape(M, K), dev)
    W, w = bf16_dev(oracle.normal(12, 2, N * K, 0.02).reshape(N, K), dev)
    b = oracle.normal(12, 3, N, 0.02) if has_b else None
    r = oracle.normal(12, 4, M * N).reshape(M, N) if has_r else None
    B = to_dev(b, dev) if has_b else None
    R = to_dev(r, dev) if has_r else None
    Y32 = torch.empty((M, N), dtype=torch.float32, device=dev)
    Y16 = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    _gemm(cbis, M, N, K, X, cbis.BF16, W, cbis.BF16, Y32, cbis.F32, bias=B, gelu=gelu, residual=R)
    _gemm(cbis, M, N, K, X, cbis.BF16, W, cbis.BF16, Y16, cbis.BF16, bias=B, gelu=gelu, residual=R)
    rows = _sample_rows(M, 512, M + 1)
    ref = oracle.gemm(x[rows], w, bias=b, gelu=gelu, residual=None if r is None else r[rows])
    # fp32 output: only accumulation order differs from the fp64 oracle
    assert np.abs(Y32.cpu().numpy()[rows] - ref).max() < FP32_TOL
    assert row_rel_err(Y16.float().cpu().numpy()[rows], ref) < LOWP_TOL


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 2048), (8192, 2048), (2048, 8192), (32000, 2048)])
def test_gemm_bf16_c4_shapes(cbis, oracle, dev, N, K):
    """Config 4's per-layer GEMMs at M=1216 (checked on sampled rows)."""
    import torch
    M = 1216
    X, x = bf16_dev(oracle.normal(13, 1, M * K).reshape(M, K), dev)
    W, w = bf16_dev(oracle.normal(13, 2, N * K, 0.02).reshape(N, K), dev)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    _gemm(cbis, M, N, K, X, cbis.BF16, W, cbis.BF16, Y, cbis.F32)
    rows = _sample_rows(M, 24, N)
    rows[-1] = M - 1  # include the ragged last M tile
    ref = oracle.gemm(x[rows], w)
    assert np.abs(Y.cpu().numpy()[rows] - ref).max() < FP32_TOL * 4


@pytest.mark.parametrize("M,xdt", [(16, "f32"), (256, "f32"), (16, "bf16"), (256, "bf16")])
def test_gemm_gelu_epilogue_accuracy(cbis, dev, M, xdt):
    """The fused GELU against fp64 erf on GEMM outputs that are exact
    (one non-zero product per output, values from -8 to 8 and around 0):
    |error| <= 1e-6 (1 + |v|), on the skinny (M=16) and tiled (M=256) paths."""
    import math
    import torch
    from helpers import sync
    N, K = 64, 64
    v = np.concatenate([np.linspace(-8, 8, M - 6), [0.0, 1e-4, -1e-4, 0.5, -0.5, 3.0]]).astype(np.float32)
    if xdt == "bf16":
        v = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    x = np.zeros((M, K), np.float32); x[:, 0] = v
    w = np.zeros((N, K), np.float32); w[:, 0] = 1.0
    dt = torch.float32 if xdt == "f32" else torch.bfloat16
    X, W = torch.from_numpy(x).to(dev).to(dt), torch.from_numpy(w).to(dev).to(dt)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    code = cbis.F32 if xdt == "f32" else cbis.BF16
    _gemm(cbis, M, N, K, X, code, W, code, Y, cbis.F32, gelu=True)
    sync()
    ref = np.array([0.5 * a * (1 + math.erf(a / math.sqrt(2))) for a in v.astype(np.float64)])
    got = Y.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ref[:, None]) <= 1e-6 * (1 + np.abs(ref[:, None])))


@pytest.mark.parametrize("wdt", ["f32", "bf16", "fp8"])
@pytest.mark.parametrize("ydt", ["f32", "bf16"])
@pytest.mark.parametrize("N,pad", [(250, 3), (252, 0), (258, 4)])
def test_gemm_parked_epilogue_ragged(cbis, oracle, dev, wdt, ydt, N, pad):
    """The LDS-parked epilogue of the single-role kernels (gemm_kernel for
    fp32 / fp8 W, gemm_bf16_dma_kernel for bf16) on ragged shapes, whole K:
    M = 600 ends inside a row tile, N = 250 / 258 inside a 4-column group
    (element-wise stores), N = 252 inside a column tile with 16-byte groups;
    Y rows padded by `pad` elements (an odd pitch forces element-wise
    stores), bias + GELU, and a residual (aliasing Y when Y is fp32),
    against the fp64 oracle; columns of the padding stay untouched."""
    import torch
    M, K = 600, 256
    ldy = N + pad
    x = oracle.normal(23, 1, M * K).reshape(M, K)
    w = oracle.normal(23, 2, N * K, 0.02).reshape(N, K)
    b = oracle.normal(23, 3, N, 0.02)
    r = oracle.normal(23, 4, M * N).reshape(M, N)
    S = None
    if wdt == "f32":
        X, W, xdt, wd, xr, wr = to_dev(x, dev), to_dev(w, dev), cbis.F32, cbis.F32, x, w
    elif wdt == "bf16":
        (X, xr), (W, wr) = bf16_dev(x, dev), bf16_dev(w, dev)
        xdt, wd = cbis.BF16, cbis.BF16
    else:
        codes, sc = oracle.quantize_e4m3_rows(w)
        (X, xr), W, S = bf16_dev(x, dev), to_dev(codes, dev), to_dev(sc, dev)
        wr = oracle.e4m3_table()[codes] * sc[:, None]
        xdt, wd = cbis.BF16, cbis.FP8E4M3
    sentinel = 7.0
    if ydt == "f32":
        Y = torch.full((M, ldy), sentinel, dtype=torch.float32, device=dev)
        Y[:, :N] = to_dev(r, dev)
        R, ldr = Y, ldy
    else:
        Y = torch.full((M, ldy), sentinel, dtype=torch.bfloat16, device=dev)
        R, ldr = to_dev(r, dev), N
    d = cbis.GemmDesc()
    d.M, d.N, d.K = M, N, K
    d.x_dtype, d.X, d.ldx = xdt, ptr(X), K
    d.w_dtype, d.W, d.ldw = wd, ptr(W), K
    d.w_scale, d.bias = ptr(S), ptr(to_dev(b, dev))
    d.epilogue = cbis.EPI_GELU
    d.residual, d.ldr = ptr(R), ldr
    d.y_dtype, d.Y, d.ldy = cbis.F32 if ydt == "f32" else cbis.BF16, ptr(Y), ldy
    cbis.check(cbis.kernels().cbis_gemm(ctypes.byref(d), stream()), "cbis_gemm")
    sync()
    got = Y.float().cpu().numpy()
    ref = oracle.gemm(xr, wr.astype(np.float32), bias=b, gelu=True, residual=r)
    tol = FP32_TOL if ydt == "f32" else 8e-3 * (1 + np.abs(ref))
    assert np.all(np.abs(got[:, :N] - ref) <= tol)
    assert np.all(got[:, N:] == sentinel)


@pytest.mark.parametrize("M", [192, 1216])
@pytest.mark.parametrize("N,K,gelu", [(2048, 4096, False), (2048, 8192, False), (1024, 4096, True), (1030, 4096, False),
                                      (2050, 4096, False), (8192, 2048, True)])
def test_gemm_bf16_split_k(cbis, oracle, dev, M, N, K, gelu):
    """Bias, GELU, and a residual that aliases Y, against the fp64 oracle, on
    the two bf16 tiled paths: grids of fewer than 128 tiles of 128 x 128
    cannot fill the GPU and split-K (fp32 partials in a caller workspace,
    reduce + epilogue) must engage, as for grids of 128-255 such tiles with
    K >= 6144 (wave-specialised 160 x 256 tiles, split-K up to 4); the
    others run the wave-specialised kernel whole-K (no workspace) with its
    row-wise epilogue: M=1216 with N=2048 or 2050 and K=4096 on 96 x 128
    tiles (ragged last M tile; N=2050 ends in a ragged column group), N=8192
    on 160 x 256 tiles parked in two row blocks (config 4's fc1 with its
    GELU)."""
    import torch
    X, x = bf16_dev(oracle.normal(15, 1, M * K).reshape(M, K), dev)
    W, w = bf16_dev(oracle.normal(15, 2, N * K, 0.02).reshape(N, K), dev)
    b = oracle.normal(15, 3, N, 0.02)
    r = None if gelu else oracle.normal(15, 4, M * N).reshape(M, N)
    B = to_dev(b, dev)
    Y = to_dev(r, dev) if r is not None else torch.empty((M, N), dtype=torch.float32, device=dev)
    used = _gemm(cbis, M, N, K, X, cbis.BF16, W, cbis.BF16, Y, cbis.F32, bias=B, gelu=gelu,
                 residual=Y if r is not None else None, workspace=True)
    t128 = -(-M // 128) * -(-N // 128)
    assert (used > 0) == (t128 < 128 or (t128 < 256 and K // 64 >= 96))
    rows = _sample_rows(M, 48, N + K)
    rows[-1] = M - 1
    ref = oracle.gemm(x[rows], w, bias=b, gelu=gelu, residual=None if r is None else r[rows])
    assert np.abs(Y.cpu().numpy()[rows] - ref).max() < FP32_TOL * 4


@pytest.mark.parametrize("M,N,K", [(1216, 2048, 8192), (192, 2048, 8192), (1216, 2048, 2048), (300, 1000, 8192),
                                   (96, 1536, 8192)])
@pytest.mark.parametrize("ln_dt", ["f32", "bf16"])
def test_gemm_layernorm_matches_gemm_then_layernorm(cbis, oracle, dev, M, N, K, ln_dt):
    """cbis_gemm_layernorm (x += h . W^T + b, then LayerNorm(x)) against
    cbis_gemm followed by cbis_layernorm on the same inputs: bit-identical x
    and normalised rows, both where K is split (the reduce and the LayerNorm
    fused: K=8192) and where it is not (K=2048); N=1000 and N=1536 end inside
    a lane chunk of the fused kernel (chunks past the row)."""
    import torch
    X, _ = bf16_dev(oracle.normal(17, 1, M * K).reshape(M, K), dev)
    W, _ = bf16_dev(oracle.normal(17, 2, N * K, 0.02).reshape(N, K), dev)
    b = to_dev(oracle.normal(17, 3, N, 0.02), dev)
    x0 = oracle.normal(17, 4, M * N).reshape(M, N)
    gam = to_dev(1.0 + oracle.normal(17, 5, N, 0.1), dev)
    bet = to_dev(oracle.normal(17, 6, N, 0.1), dev)
    code = cbis.F32 if ln_dt == "f32" else cbis.BF16
    tdt = torch.float32 if ln_dt == "f32" else torch.bfloat16
    outs = []
    for fused in (True, False):
        Y = to_dev(x0, dev)
        d = cbis.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.x_dtype, d.X, d.ldx = cbis.BF16, ptr(X), K
        d.w_dtype, d.W, d.ldw = cbis.BF16, ptr(W), K
        d.bias = ptr(b)
        d.residual, d.ldr = ptr(Y), N
        d.y_dtype, d.Y, d.ldy = cbis.F32, ptr(Y), N
        need = cbis.kernels().cbis_gemm_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
        d.workspace, d.workspace_bytes = ptr(ws), need
        ln = torch.empty((M, N), dtype=tdt, device=dev)
        if fused:
            cbis.check(cbis.kernels().cbis_gemm_layernorm(ctypes.byref(d), ptr(gam), ptr(bet), 1e-5, code, ptr(ln), N,
                                                           stream()), "cbis_gemm_layernorm")
        else:
            cbis.check(cbis.kernels().cbis_gemm(ctypes.byref(d), stream()), "cbis_gemm")
            cbis.check(cbis.kernels().cbis_layernorm(M, N, ptr(Y), N, ptr(gam), ptr(bet), 1e-5, code, ptr(ln), N,
                                                     stream()), "cbis_layernorm")
        sync()
        outs.append((Y.cpu().numpy().view(np.uint32), ln.view(torch.int16 if ln_dt == "bf16" else torch.int32).cpu().numpy()))
        if fused:
            split = need > 0
    assert split == (K == 8192)
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("wdt", ["bf16", "fp8"])
@pytest.mark.parametrize("M,N,K,parts", [(16, 2048, 8192, (4, 4)), (16, 2048, 2048, (4, 2)), (1, 2048, 8192, (4, 4)),
                                         (64, 2048, 8192, (4, 4)), (33, 1000, 4096, (4, 4)),
                                         (16, 6144, 2048, (1, 1))])
def test_gemm_layernorm_skinny_split(cbis, oracle, dev, M, N, K, parts, wdt):
    """Decode-sized cbis_gemm_layernorm (config 5's out-projection and fc2:
    x += h . W^T * scale + b, then LayerNorm(x)): the skinny kernel splits K
    into `parts` ranges (its 16-column workgroups alone would not occupy the
    CUs) and the partials are summed, scaled, biased and added to the
    residual in the LayerNorm's kernel.  x against the fp64 oracle
    (1e-5 relative), the normalised rows against the oracle's LayerNorm of
    the GPU's x (one bf16 rounding), and both against the unsplit cbis_gemm
    then cbis_layernorm (summation order only)."""
    import torch
    K_ = cbis.kernels()
    parts = parts[0] if wdt == "bf16" else parts[1]  # every wave keeps >= 2 MFMA k steps (32 / 64 k)
    x = oracle.normal(19, 1, M * K).reshape(M, K)
    w = oracle.normal(19, 2, N * K, 0.02).reshape(N, K)
    b = oracle.normal(19, 3, N, 0.02)
    x0 = oracle.normal(19, 4, M * N).reshape(M, N)
    gam = 1.0 + oracle.normal(19, 5, N, 0.1)
    bet = oracle.normal(19, 6, N, 0.1)
    X, xv = bf16_dev(x, dev)
    if wdt == "bf16":
        W, wv = bf16_dev(w, dev)
        S, sc = None, None
        wd = cbis.BF16
    else:
        codes, sc = oracle.quantize_e4m3_rows(w)
        W, S, wv, wd = to_dev(codes, dev), to_dev(sc, dev), oracle.e4m3_table()[codes], cbis.FP8E4M3
    B, G, Be = to_dev(b, dev), to_dev(gam, dev), to_dev(bet, dev)
    outs = []
    for fused in (True, False):
        Y = to_dev(x0, dev)
        d = cbis.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.x_dtype, d.X, d.ldx = cbis.BF16, ptr(X), K
        d.w_dtype, d.W, d.ldw, d.w_scale = wd, ptr(W), K, ptr(S)
        d.bias = ptr(B)
        d.residual, d.ldr = ptr(Y), N
        d.y_dtype, d.Y, d.ldy = cbis.F32, ptr(Y), N
        need = K_.cbis_gemm_layernorm_workspace_size(ctypes.byref(d))
        assert need == (parts * M * N * 4 if parts > 1 else 0)
        if wdt == "fp8" or M <= 32:  # plain cbis_gemm keeps the skinny kernel whole (bf16 x bf16 calls of
            assert K_.cbis_gemm_workspace_size(ctypes.byref(d)) == 0  # 33..64 rows take the tiles)
        ws = torch.empty(max(4, need // 4), dtype=torch.float32, device=dev)
        d.workspace, d.workspace_bytes = ptr(ws), need
        ln = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if fused:
            cbis.check(K_.cbis_gemm_layernorm(ctypes.byref(d), ptr(G), ptr(Be), 1e-5, cbis.BF16, ptr(ln), N,
                                              stream()), "cbis_gemm_layernorm")
        else:
            d.workspace, d.workspace_bytes = None, 0
            cbis.check(K_.cbis_gemm(ctypes.byref(d), stream()), "cbis_gemm")
            cbis.check(K_.cbis_layernorm(M, N, ptr(Y), N, ptr(G), ptr(Be), 1e-5, cbis.BF16, ptr(ln), N, stream()),
                       "cbis_layernorm")
        sync()
        outs.append((Y.cpu().numpy(), ln.float().cpu().numpy()))
    ref = oracle.gemm(xv, wv, w_scale=sc, bias=b, residual=x0)
    for got, lnv in outs:
        assert (np.abs(got - ref) / (1.0 + np.abs(ref))).max() < 1e-5
        lref = oracle.layernorm(got, gam, bet)
        assert (np.abs(lnv - lref) / (1.0 + np.abs(lref))).max() < 2 ** -7
    assert (np.abs(outs[0][0] - outs[1][0]) / (1.0 + np.abs(outs[1][0]))).max() < 1e-5


@pytest.mark.parametrize("wdt", ["f32", "bf16", "fp8"])
@pytest.mark.parametrize("M,K", [(1, 256), (8, 256), (33, 512), (64, 512), (16, 2048), (100, 256), (8, 4096)])
def test_layernorm_gemm_matches_layernorm_then_gemm(cbis, oracle, dev, M, K, wdt):
    """cbis_layernorm_gemm (Y = LayerNorm(x) . W^T + b, GELU) against
    cbis_layernorm into X followed by cbis_gemm: bit-identical Y where both
    GEMMs run on the same kernel (bf16 x bf16 plain calls of 33..64 rows run
    on the tiles: within fp32 rounding there).  Decode-sized
    calls with short rows (M <= 64, K <= 512) form the normalised rows inside
    the skinny GEMM (X is then left untouched); M = 100 and K = 2048 / 4096
    take the two-kernel path."""
    import torch
    N = 200
    x = oracle.normal(23, 1, M * K).reshape(M, K) * 2.0 + 0.5
    gam = to_dev(1.0 + oracle.normal(23, 5, K, 0.1), dev)
    bet = to_dev(oracle.normal(23, 6, K, 0.1), dev)
    b = to_dev(oracle.normal(23, 3, N, 0.02), dev)
    w = oracle.normal(23, 2, N * K, 0.02).reshape(N, K)
    xd = to_dev(x, dev)
    if wdt == "f32":
        W, S, xdt, wd = to_dev(w, dev), None, cbis.F32, cbis.F32
    elif wdt == "bf16":
        (W, _), S, xdt, wd = bf16_dev(w, dev), None, cbis.BF16, cbis.BF16
    else:
        codes, sc = oracle.quantize_e4m3_rows(w)
        W, S, xdt, wd = to_dev(codes, dev), to_dev(sc, dev), cbis.BF16, cbis.FP8E4M3
    tdt = torch.float32 if xdt == cbis.F32 else torch.bfloat16
    outs = []
    for fused in (True, False):
        Xbuf = torch.full((M, K), 7.0, dtype=tdt, device=dev)
        Y = torch.empty((M, N), dtype=torch.float32, device=dev)
        d = cbis.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.x_dtype, d.X, d.ldx = xdt, ptr(Xbuf), K
        d.w_dtype, d.W, d.ldw = wd, ptr(W), K
        d.w_scale, d.bias = ptr(S), ptr(b)
        d.epilogue = cbis.EPI_GELU
        d.y_dtype, d.Y, d.ldy = cbis.F32, ptr(Y), N
        if fused:
            cbis.check(cbis.kernels().cbis_layernorm_gemm(ctypes.byref(d), ptr(xd), K, ptr(gam), ptr(bet), 1e-5,
                                                           stream()), "cbis_layernorm_gemm")
        else:
            cbis.check(cbis.kernels().cbis_layernorm(M, K, ptr(xd), K, ptr(gam), ptr(bet), 1e-5, xdt, ptr(Xbuf), K,
                                                     stream()), "cbis_layernorm")
            cbis.check(cbis.kernels().cbis_gemm(ctypes.byref(d), stream()), "cbis_gemm")
        sync()
        outs.append(Y.cpu().numpy().view(np.uint32))
        if fused:
            # the prologue path leaves X untouched; the two-kernel path writes LayerNorm(x) there
            untouched = bool((Xbuf.float() == 7.0).all())
            assert untouched == (M <= 64 and K <= 512), (M, K)
    if wdt == "bf16" and 32 < M <= 64:
        # The plain bf16 x bf16 GEMM of 33..64 rows runs on the tiles, which
        # sum in another order than the skinny kernel: fp32 rounding apart.
        a, b_ = outs[0].view(np.float32), outs[1].view(np.float32)
        assert (np.abs(a - b_) / (1.0 + np.abs(b_))).max() < 1e-5
    else:
        assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("wdt", ["f32", "bf16", "fp8"])
@pytest.mark.parametrize("M,K", [(8, 256), (64, 512), (16, 2048), (100, 256)])
def test_layernorm_gemm_argmax_matches_layernorm_then_argmax(cbis, oracle, dev, M, K, wdt):
    """cbis_layernorm_gemm_argmax against cbis_layernorm into X followed by
    cbis_gemm_argmax: identical tokens and bit-identical margins, whether the
    LayerNorm runs inside the skinny GEMM (M <= 64, K <= 512) or before it."""
    import torch
    K_ = cbis.kernels()
    N = 1000
    x = oracle.normal(29, 1, M * K).reshape(M, K) * 1.5 - 0.25
    gam = to_dev(1.0 + oracle.normal(29, 5, K, 0.1), dev)
    bet = to_dev(oracle.normal(29, 6, K, 0.1), dev)
    w = oracle.normal(29, 2, N * K, 0.02).reshape(N, K)
    b = to_dev(oracle.normal(29, 3, N, 0.02), dev)
    xd = to_dev(x, dev)
    if wdt == "f32":
        W, S, xdt, wd = to_dev(w, dev), None, cbis.F32, cbis.F32
    elif wdt == "bf16":
        (W, _), S, xdt, wd = bf16_dev(w, dev), None, cbis.BF16, cbis.BF16
    else:
        codes, sc = oracle.quantize_e4m3_rows(w)
        W, S, xdt, wd = to_dev(codes, dev), to_dev(sc, dev), cbis.BF16, cbis.FP8E4M3
    tdt = torch.float32 if xdt == cbis.F32 else torch.bfloat16
    res = []
    for fused in (True, False):
        Xbuf = torch.zeros((M, K), dtype=tdt, device=dev)
        d = cbis.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.x_dtype, d.X, d.ldx = xdt, ptr(Xbuf), K
        d.w_dtype, d.W, d.ldw = wd, ptr(W), K
        d.w_scale, d.bias = ptr(S), ptr(b)
        need = K_.cbis_gemm_argmax_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(4, need // 4), dtype=torch.float32, device=dev)
        nxt = torch.full((M,), -1, dtype=torch.int32, device=dev)
        mar = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
        if fused:
            cbis.check(K_.cbis_layernorm_gemm_argmax(ctypes.byref(d), ptr(xd), K, ptr(gam), ptr(bet), 1e-5, ptr(nxt),
                                                     ptr(mar), ptr(ws), need, stream()), "cbis_layernorm_gemm_argmax")
        else:
            cbis.check(K_.cbis_layernorm(M, K, ptr(xd), K, ptr(gam), ptr(bet), 1e-5, xdt, ptr(Xbuf), K, stream()),
                       "cbis_layernorm")
            cbis.check(K_.cbis_gemm_argmax(ctypes.byref(d), ptr(nxt), ptr(mar), ptr(ws), need, stream()),
                       "cbis_gemm_argmax")
        sync()
        res.append((nxt.cpu().numpy(), mar.cpu().numpy().view(np.uint32)))
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1], res[1][1])
    assert (res[0][0] >= 0).all() and (res[0][0] < N).all()


@pytest.mark.parametrize("M", [16, 200])
def test_gemm_fp8_weights(cbis, oracle, dev, M):
    import torch
    N, K = 1000, 2048
    w = oracle.normal(14, 2, N * K, 0.02).reshape(N, K)
    codes, sc = oracle.quantize_e4m3_rows(w)
    wdq = oracle.e4m3_table()[codes]
    X, x = bf16_dev(oracle.normal(14, 1, M * K).reshape(M, K), dev)
    b = oracle.normal(14, 3, N, 0.02)
    C, S, B = to_dev(codes, dev), to_dev(sc, dev), to_dev(b, dev)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    _gemm(cbis, M, N, K, X, cbis.BF16, C, cbis.FP8E4M3, Y, cbis.F32, bias=B, w_scale=S)
    ref = oracle.gemm(x, wdq, w_scale=sc, bias=b)
    assert np.abs(Y.cpu().numpy() - ref).max() < FP32_TOL


def test_gemm_fp8_decode_every_code(cbis, oracle, dev):
    """Every OCP e4m3 code through the decode-sized (skinny) GEMM: row n of W
    holds code n at k = 0 and zeros elsewhere, X = e_0, scale 1, so
    Y[0, n] is the decoded code itself -- exactly the oracle's table value
    (NaN codes 0x7F / 0xFF must decode to NaN)."""
    import torch
    N, K = 256, 64
    codes = np.zeros((N, K), np.uint8)
    codes[:, 0] = np.arange(256, dtype=np.uint8)
    x = np.zeros((1, K), np.float32)
    x[0, 0] = 1.0
    X, _ = bf16_dev(x, dev)
    C, S = to_dev(codes, dev), to_dev(np.ones(N, np.float32), dev)
    Y = torch.empty((1, N), dtype=torch.float32, device=dev)
    _gemm(cbis, 1, N, K, X, cbis.BF16, C, cbis.FP8E4M3, Y, cbis.F32, w_scale=S)
    got = Y.cpu().numpy()[0]
    ref = oracle.e4m3_table()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    # exact equality of every value (the accumulator turns 1 * -0 into +0,
    # so code 0x80 compares equal to 0 rather than bit for bit)
    bad = [hex(c) for c in range(256) if not nan[c] and got[c] != ref[c]]
    assert not bad, bad


@pytest.mark.parametrize("M", [1, 8, 16, 33, 64])
@pytest.mark.parametrize("wdt", ["f32", "bf16", "fp8"])
def test_gemm_skinny_decode_rows(cbis, oracle, dev, M, wdt):
    """Decode-sized M for every weight dtype (the weight-streaming kernel;
    bf16 x bf16 calls of 33..64 rows the direct-to-LDS tiles), with bias +
    GELU and with bias + a residual aliasing Y, against the oracle."""
    import torch
    N, K = 1040, 1024  # N not a multiple of the 16-column tile
    w = oracle.normal(16, 2, N * K, 0.02).reshape(N, K)
    xf = oracle.normal(16, 1, M * K).reshape(M, K)
    b = oracle.normal(16, 3, N, 0.02)
    r = oracle.normal(16, 4, M * N).reshape(M, N)
    sc = None
    if wdt == "f32":
        X, x = to_dev(xf, dev), xf
        W, wq, xdt, wdt_c = to_dev(w, dev), w, cbis.F32, cbis.F32
    else:
        X, x = bf16_dev(xf, dev)
        xdt = cbis.BF16
        if wdt == "bf16":
            W, wq = bf16_dev(w, dev)
            wdt_c = cbis.BF16
        else:
            codes, sc = oracle.quantize_e4m3_rows(w)
            W, wq, wdt_c = to_dev(codes, dev), oracle.e4m3_table()[codes], cbis.FP8E4M3
    S = to_dev(sc, dev) if sc is not None else None
    B = to_dev(b, dev)
    Yg = torch.empty((M, N), dtype=torch.float32, device=dev)
    _gemm(cbis, M, N, K, X, xdt, W, wdt_c, Yg, cbis.F32, bias=B, w_scale=S, gelu=True)
    Yr = to_dev(r, dev)
    _gemm(cbis, M, N, K, X, xdt, W, wdt_c, Yr, cbis.F32, bias=B, w_scale=S, residual=Yr)
    ref_g = oracle.gemm(x, wq, w_scale=sc, bias=b, gelu=True)
    ref_r = oracle.gemm(x, wq, w_scale=sc, bias=b, residual=r)
    assert np.abs(Yg.cpu().numpy() - ref_g).max() < FP32_TOL
    assert np.abs(Yr.cpu().numpy() - ref_r).max() < FP32_TOL


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_gemm_qkv_scatter_epilogue(cbis, oracle, dev, kv_dtype):
    """Fused QKV projection: Q to its buffer, K/V straight into page slots
    (the fused form of scatter_kv_to_cache, kernels/attention.cu:7-19)."""
    import torch
    M, D, P = 77, 256, 40
    dt = cbis.F32 if kv_dtype == "f32" else cbis.BF16
    act = np.float32
    x = oracle.normal(15, 1, M * D).reshape(M, D)
    w = oracle.normal(15, 2, 3 * D * D, 0.02).reshape(3 * D, D)
    b = oracle.normal(15, 3, 3 * D, 0.02)
    if dt == cbis.F32:
        X, W = to_dev(x, dev), to_dev(w, dev)
        xv, wv = x, w
        tdt = torch.float32
    else:
        X, xv = bf16_dev(x, dev)
        W, wv = bf16_dev(w, dev)
        tdt = torch.bfloat16
    slots = rng(5).permutation(P * 16)[:M]
    wpage, woff = (slots // 16).astype(np.int32), (slots % 16).astype(np.int32)
    kp = torch.zeros((P, 16, D), dtype=tdt, device=dev)
    vp = torch.zeros((P, 16, D), dtype=tdt, device=dev)
    Q = torch.zeros((M, D), dtype=torch.float32, device=dev)
    kv = {"col0": D, "width": D, "dtype": dt, "k": kp, "v": vp, "wpage": to_dev(wpage, dev),
          "woff": to_dev(woff, dev), "ldy": D}
    _gemm(cbis, M, 3 * D, D, X, dt, W, dt, Q, cbis.F32, bias=to_dev(b, dev), kv=kv)
    ref = oracle.gemm(xv, wv, bias=b).astype(act)
    assert np.abs(Q.cpu().numpy() - ref[:, :D]).max() < FP32_TOL
    kh, vh = kp.float().cpu().numpy(), vp.float().cpu().numpy()
    gk, gv = kh[wpage, woff], vh[wpage, woff]
    if dt == cbis.F32:
        assert np.abs(gk - ref[:, D:2 * D]).max() < FP32_TOL
        assert np.abs(gv - ref[:, 2 * D:]).max() < FP32_TOL
    else:
        assert row_rel_err(gk, ref[:, D:2 * D]) < LOWP_TOL
        assert row_rel_err(gv, ref[:, 2 * D:]) < LOWP_TOL
    # untouched slots stay zero
    mask = np.ones((P, 16), bool)
    mask[wpage, woff] = False
    assert not kh[mask].any() and not vh[mask].any()


@pytest.mark.parametrize("M,D", [(700, 1024), (1216, 2048)])
@pytest.mark.parametrize("ydt", ["f32", "bf16"])
def test_gemm_qkv_scatter_epilogue_wave_specialised(cbis, oracle, dev, M, D, ydt):
    """The fused QKV projection at sizes that run the wave-specialised kernel
    (M=700, d=1024: 96 x 128 tiles; M=1216, d=2048: config 4, 128 x 256
    tiles): bf16 K/V straight into page slots, Q in fp32 or bf16, through the
    row-wise epilogue."""
    import torch
    P = M // 16 + 8
    x = oracle.normal(16, 1, M * D).reshape(M, D)
    w = oracle.normal(16, 2, 3 * D * D, 0.02).reshape(3 * D, D)
    b = oracle.normal(16, 3, 3 * D, 0.02)
    X, xv = bf16_dev(x, dev)
    W, wv = bf16_dev(w, dev)
    slots = rng(6).permutation(P * 16)[:M]
    wpage, woff = (slots // 16).astype(np.int32), (slots % 16).astype(np.int32)
    kp = torch.zeros((P, 16, D), dtype=torch.bfloat16, device=dev)
    vp = torch.zeros((P, 16, D), dtype=torch.bfloat16, device=dev)
    qdt = torch.float32 if ydt == "f32" else torch.bfloat16
    Q = torch.zeros((M, D), dtype=qdt, device=dev)
    kv = {"col0": D, "width": D, "dtype": cbis.BF16, "k": kp, "v": vp, "wpage": to_dev(wpage, dev),
          "woff": to_dev(woff, dev), "ldy": D}
    _gemm(cbis, M, 3 * D, D, X, cbis.BF16, W, cbis.BF16, Q, cbis.F32 if ydt == "f32" else cbis.BF16,
          bias=to_dev(b, dev), kv=kv)
    ref = oracle.gemm(xv, wv, bias=b)
    q = Q.float().cpu().numpy()
    if ydt == "f32":
        assert np.abs(q - ref[:, :D]).max() < FP32_TOL * 4
    else:
        assert row_rel_err(q, ref[:, :D]) < LOWP_TOL
    kh, vh = kp.float().cpu().numpy(), vp.float().cpu().numpy()
    assert row_rel_err(kh[wpage, woff], ref[:, D:2 * D]) < LOWP_TOL
    assert row_rel_err(vh[wpage, woff], ref[:, 2 * D:]) < LOWP_TOL
    mask = np.ones((P, 16), bool)
    mask[wpage, woff] = False
    assert not kh[mask].any() and not vh[mask].any()


def test_gemm_rejects_bad_shapes(cbis):
    d = cbis.GemmDesc()
    d.M, d.N, d.K = 4, 8, 100  # K not a multiple of 64 for bf16
    d.x_dtype = d.w_dtype = d.y_dtype = cbis.BF16
    d.X = d.W = d.Y = 256
    d.ldx = d.ldw = 100
    d.ldy = 8
    assert cbis.kernels().cbis_gemm(ctypes.byref(d), None) == 2


# --------------------------------------------------------------------------
# LayerNorm, embedding, argmax, reference elementwise launchers
# --------------------------------------------------------------------------

@pytest.mark.parametrize("D", [256, 2048])
@pytest.mark.parametrize("ydt", ["f32", "bf16"])
def test_layernorm(cbis, oracle, dev, D, ydt):
    import torch
    M = 300
    x = (oracle.normal(16, 1, M * D).reshape(M, D) * 3 + 1.5).astype(np.float32)
    g = (1 + oracle.normal(16, 2, D, 0.3)).astype(np.float32)
    b = oracle.normal(16, 3, D, 0.3)
    X, G, B = to_dev(x, dev), to_dev(g, dev), to_dev(b, dev)
    tdt = torch.float32 if ydt == "f32" else torch.bfloat16
    Y = torch.empty((M, D), dtype=tdt, device=dev)
    cbis.check(cbis.kernels().cbis_layernorm(M, D, ptr(X), D, ptr(G), ptr(B), 1e-5, cbis.DTYPES[ydt], ptr(Y), D,
                                             stream()))
    sync()
    ref = oracle.layernorm(x, g, b)
    if ydt == "f32":
        assert np.abs(Y.cpu().numpy() - ref).max() < 1e-5 * 10
    else:
        assert row_rel_err(Y.float().cpu().numpy(), ref) < LOWP_TOL


@pytest.mark.parametrize("edt", ["f32", "bf16"])
def test_embed(cbis, oracle, dev, edt):
    import torch
    V, S, D, M = 512, 100, 256, 50
    te = oracle.normal(17, 1, V * D, 0.02).reshape(V, D)
    pe = oracle.normal(17, 2, S * D, 0.02).reshape(S, D)
    tok = oracle.uniform_int(17, 3, M, 0, V - 1)
    pos = oracle.uniform_int(17, 4, M, 0, S - 1)
    if edt == "f32":
        TE, PE, tev, pev = to_dev(te, dev), to_dev(pe, dev), te, pe
    else:
        (TE, tev), (PE, pev) = bf16_dev(te, dev), bf16_dev(pe, dev)
    out = torch.empty((M, D), dtype=torch.float32, device=dev)
    TOK, POS = to_dev(tok, dev), to_dev(pos, dev)  # keep the device copies alive until the launch completes
    cbis.check(cbis.kernels().cbis_embed(M, D, ptr(TOK), ptr(POS), cbis.DTYPES[edt], ptr(TE), ptr(PE), V, S,
                                         ptr(out), stream()))
    sync()
    ref = tev[tok].astype(np.float64) + pev[pos]
    assert np.array_equal(out.cpu().numpy(), ref.astype(np.float32))
    # ids outside the tables read nothing: those rows come out NaN, the rest exact
    bad_tok, bad_pos = tok.copy(), pos.copy()
    bad_tok[[3, 9]] = [V, -1]
    bad_pos[[20, 41]] = [S, -7]
    TOK, POS = to_dev(bad_tok, dev), to_dev(bad_pos, dev)
    out.fill_(0.0)
    cbis.check(cbis.kernels().cbis_embed(M, D, ptr(TOK), ptr(POS), cbis.DTYPES[edt], ptr(TE), ptr(PE), V, S,
                                         ptr(out), stream()))
    sync()
    got = out.cpu().numpy()
    bad = np.zeros(M, bool)
    bad[[3, 9, 20, 41]] = True
    assert np.isnan(got[bad]).all()
    assert np.array_equal(got[~bad], ref.astype(np.float32)[~bad])


@pytest.mark.parametrize("edt", ["f32", "bf16"])
@pytest.mark.parametrize("stage_words", [0, 1, 777, 70000])
def test_embed_from_token_src_and_staging(cbis, oracle, dev, edt, stage_words):
    """cbis_embed_from: rows with token_src >= 0 take src_tokens[token_src]
    (ids out of range there still give NaN rows), the others token_ids; the
    same launch copies stage_words 16-byte words (here device to device; the
    runner's host-memory case is covered by its whole-step tests) and
    touches nothing past them.  Misaligned or unpaired arguments are
    rejected."""
    import torch
    V, S, D, M = 512, 100, 256, 50
    te = oracle.normal(19, 1, V * D, 0.02).reshape(V, D)
    pe = oracle.normal(19, 2, S * D, 0.02).reshape(S, D)
    tok = oracle.uniform_int(19, 3, M, 0, V - 1)
    pos = oracle.uniform_int(19, 4, M, 0, S - 1)
    prev = oracle.uniform_int(19, 5, 20, 0, V - 1)
    prev[7] = V + 3  # an out-of-range token left by the previous step
    rng = np.random.default_rng(19)
    tsrc = np.where(rng.random(M) < 0.6, rng.integers(0, 20, M), -1).astype(np.int32)
    tsrc[0], tsrc[1] = 7, -1
    tok[tsrc >= 0] = -5  # not read for those rows
    if edt == "f32":
        TE, PE, tev, pev = to_dev(te, dev), to_dev(pe, dev), te, pe
    else:
        (TE, tev), (PE, pev) = bf16_dev(te, dev), bf16_dev(pe, dev)
    out = torch.empty((M, D), dtype=torch.float32, device=dev)
    TOK, POS, TSRC, PREV = to_dev(tok, dev), to_dev(pos, dev), to_dev(tsrc, dev), to_dev(prev, dev)
    src_words = torch.randint(-2 ** 31, 2 ** 31 - 1, (max(stage_words, 1) * 4,), dtype=torch.int32, device=dev)
    dst_words = torch.full(((stage_words + 8) * 4,), 12345, dtype=torch.int32, device=dev)
    k = cbis.kernels()
    cbis.check(k.cbis_embed_from(M, D, ptr(TOK), ptr(TSRC), ptr(PREV), ptr(POS), cbis.DTYPES[edt], ptr(TE), ptr(PE),
                                 V, S, ptr(out), ptr(src_words), ptr(dst_words), stage_words * 16, stream()))
    sync()
    used = np.where(tsrc >= 0, prev[np.maximum(tsrc, 0)], tok)
    bad = used >= V
    ref = tev[np.where(bad, 0, used)].astype(np.float64) + pev[pos]
    got = out.cpu().numpy()
    assert bad[0] and np.isnan(got[bad]).all()
    assert np.array_equal(got[~bad], ref.astype(np.float32)[~bad])
    d = dst_words.cpu().numpy()
    assert np.array_equal(d[: stage_words * 4], src_words.cpu().numpy()[: stage_words * 4])
    assert (d[stage_words * 4:] == 12345).all()
    # 8 bytes is not a 16-byte multiple; an offset of 4 bytes is misaligned;
    # token_src without src_tokens is unpaired.
    assert k.cbis_embed_from(M, D, ptr(TOK), ptr(TSRC), ptr(PREV), ptr(POS), cbis.DTYPES[edt], ptr(TE), ptr(PE), V,
                             S, ptr(out), ptr(src_words), ptr(dst_words), 8, stream()) != 0
    assert k.cbis_embed_from(M, D, ptr(TOK), ptr(TSRC), ptr(PREV), ptr(POS), cbis.DTYPES[edt], ptr(TE), ptr(PE), V,
                             S, ptr(out), ptr(src_words) + 4, ptr(dst_words), 16, stream()) != 0
    assert k.cbis_embed_from(M, D, ptr(TOK), ptr(TSRC), None, ptr(POS), cbis.DTYPES[edt], ptr(TE), ptr(PE), V,
                             S, ptr(out), None, None, 0, stream()) != 0


@pytest.mark.parametrize("N", [32000, 1001, 4 * 1024 * 9 + 12])
def test_argmax_first_max_wins(cbis, oracle, dev, N):
    """Both load paths (16-byte rows in unrolled float4 rounds plus a tail,
    and the scalar path for an odd width) against the sequential scan."""
    import torch
    M = 64
    L = oracle.normal(18, 1, M * N).reshape(M, N)
    L[0, :] = 1.0                   # all equal -> 0
    L[1, 5] = L[1, N - 1] = 99.0    # tie -> 5
    L[2, :] = -np.inf               # -inf row -> 0
    L[3, N - 1] = 50.0              # last column
    T = to_dev(L, dev)
    out = torch.empty(M, dtype=torch.int32, device=dev)
    cbis.check(cbis.kernels().cbis_argmax_rows(M, N, ptr(T), N, ptr(out), stream()))
    sync()
    assert np.array_equal(out.cpu().numpy(), oracle.argmax_rows(L))


def test_reference_signature_elementwise(cbis, oracle, dev):
    import torch
    K = cbis.kernels()
    T, D, V, S = 40, 256, 1000, 64
    te = oracle.normal(19, 1, V * D, 0.02).reshape(V, D)
    pe = oracle.normal(19, 2, S * D, 0.02).reshape(S, D)
    tok = oracle.uniform_int(19, 3, T, 0, V - 1)
    pos = np.arange(T, dtype=np.int32)
    x = torch.empty((T, D), dtype=torch.float32, device=dev)
    # device copies are bound to names so they outlive the asynchronous launches
    TOK, POS, TE, PE = to_dev(tok, dev), to_dev(pos, dev), to_dev(te, dev), to_dev(pe, dev)
    cbis.check(K.cbis_embed_lookup_add(ptr(TOK), ptr(POS), ptr(TE), ptr(PE), ptr(x), T, D, stream()))
    g = (1 + oracle.normal(19, 4, D, 0.1)).astype(np.float32)
    b = oracle.normal(19, 5, D, 0.1)
    y = torch.empty_like(x)
    G, B = to_dev(g, dev), to_dev(b, dev)
    cbis.check(K.cbis_layernorm_forward(ptr(x), ptr(G), ptr(B), ptr(y), T, D, stream()))
    w = oracle.normal(19, 6, 1024 * D, 0.02).reshape(1024, D)
    bb = oracle.normal(19, 7, 1024, 0.02)
    h = torch.empty((T, 1024), dtype=torch.float32, device=dev)
    W, BB = to_dev(w, dev), to_dev(bb, dev)
    cbis.check(K.cbis_linear_forward(ptr(y), ptr(W), ptr(BB), ptr(h), T, D, 1024, stream()))
    cbis.check(K.cbis_gelu_forward(ptr(h), T, 1024, stream()))
    r = torch.ones((T, 1024), dtype=torch.float32, device=dev)
    cbis.check(K.cbis_residual_add(ptr(r), ptr(h), T, 1024, stream()))
    sync()
    xe = te[tok].astype(np.float64) + pe[pos]
    assert np.abs(x.cpu().numpy() - xe).max() < 1e-7
    ye = oracle.layernorm(xe.astype(np.float32), g, b)
    assert np.abs(y.cpu().numpy() - ye).max() < 1e-4
    he = oracle.gemm(y.cpu().numpy(), w, bias=bb, gelu=True)
    assert np.abs(r.cpu().numpy() - (1.0 + he)).max() < FP32_TOL


# --------------------------------------------------------------------------
# Paged attention
# --------------------------------------------------------------------------

def _attn_desc(cbis, n_rows, H, q, kp, vp, num_pages, bt, bt_stride, pos, out, kv_dtype, q_dtype=0, out_dtype=0,
               rows=None, row_bt=None, max_kv=0, split=0, ws=None):
    d = cbis.AttnDesc()
    d.n_rows, d.rows, d.n_heads, d.head_dim, d.page_size = n_rows, ptr(rows), H, 32, 16
    d.q_dtype, d.q, d.ldq = q_dtype, ptr(q), H * 32
    d.kv_dtype, d.k_pool, d.v_pool, d.num_pages = kv_dtype, ptr(kp), ptr(vp), num_pages
    d.block_table, d.bt_stride, d.row_bt, d.row_pos = ptr(bt), bt_stride, ptr(row_bt), ptr(pos)
    d.out_dtype, d.out, d.ldo = out_dtype, ptr(out), H * 32
    d.max_kv_len, d.split_tokens = max_kv, split
    if ws is not None:
        d.workspace, d.workspace_bytes = ptr(ws), ws.numel() * ws.element_size()
    # The descriptor holds raw device addresses: keep every tensor it points
    # to alive as long as the descriptor (a temporary freed here could be
    # handed to the next allocation, e.g. the workspace, while a kernel still
    # reads it through the descriptor).
    d.keep_alive = (q, kp, vp, bt, pos, out, rows, row_bt, ws)
    return d


def _c3_inputs(oracle, n_seq=256, lo=128, hi=2048, pool=40000, seed=0):
    """Config 3: kv_len U[lo, hi], one query per sequence at pos kv_len-1,
    a random permutation of a pool of `pool` pages as the page table."""
    kv = oracle.uniform_int(seed, 3001, n_seq, lo, hi)
    npages = (kv + 15) // 16
    perm = rng(seed).permutation(pool).astype(np.int32)
    stride = int(npages.max())
    bt = np.zeros((n_seq, stride), np.int32)
    off = 0
    for i in range(n_seq):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    assert off <= pool
    return kv.astype(np.int32), bt


@pytest.mark.parametrize("page_size", [1, 3, 8, 16, 32, 64])
def test_fused_attention_twin_any_page_size(cbis, oracle, dev, page_size):
    """The reference signature takes page_size at run time
    (include/attention.hpp:29-33).  Rows of kv 1, a page boundary either side,
    a few chunks of 64 keys and 300; 5 heads; a permuted pool; rows 2 and 3
    share a sequence's table; one row attends with pos past its table's
    capacity (kv clamped to pages_per_seq * page_size, as the page_size 16
    path clamps).  Against the fp64 oracle at the same page size."""
    import torch
    H, HD = 5, 32
    kv = np.array([1, page_size, page_size + 1, 64, 65, 129, 300], np.int32)
    S = kv.size
    npages = (kv + page_size - 1) // page_size
    stride = int(npages.max())
    P = int(npages.sum()) + 7
    perm = rng(page_size).permutation(P).astype(np.int32)
    bt = np.zeros((S, stride), np.int32)
    off = 0
    for i in range(S):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    bt[3] = bt[2]  # row 3 reads row 2's sequence at a later position...
    kv[3] = kv[2] + 3 if kv[2] + 3 <= npages[2] * page_size else kv[2]
    pos = kv - 1
    pos_dev = pos.copy()
    pos_dev[-1] = stride * page_size + 50  # ...and the last row asks past its table
    g = rng(100 + page_size)
    kpool = g.standard_normal((P, page_size, H, HD)).astype(np.float32)
    vpool = g.standard_normal((P, page_size, H, HD)).astype(np.float32)
    q = g.standard_normal((S, H * HD)).astype(np.float32)
    out = torch.full((S, H * HD), 7.0, dtype=torch.float32, device=dev)
    K = cbis.kernels()
    QD, KD, VD = to_dev(q, dev), to_dev(kpool, dev), to_dev(vpool, dev)
    BT, POS = to_dev(bt, dev), to_dev(pos_dev.astype(np.int32), dev)
    cbis.check(K.cbis_fused_paged_causal_attention(ptr(QD), ptr(KD), ptr(VD), ptr(BT), ptr(POS), ptr(out), S, H, HD,
                                                   page_size, stride, stream()))
    sync()
    pos_ref = pos.copy()
    pos_ref[-1] = stride * page_size - 1  # the clamp
    ref = oracle.paged_attention(q, kpool, vpool, bt, pos_ref, H, HD, page_size)
    assert np.abs(out.cpu().numpy() - ref).max() < FP32_TOL
    # the single-key row is exactly its V
    assert np.abs(out.cpu().numpy()[0] - vpool[bt[0, 0], 0].reshape(-1)).max() < 1e-6


def test_fused_attention_twin_rejects_bad_page_size(cbis, dev):
    import torch
    x = torch.zeros(64, dtype=torch.float32, device=dev)
    i = torch.zeros(4, dtype=torch.int32, device=dev)
    K = cbis.kernels()
    for ps in (0, -16):
        rc = K.cbis_fused_paged_causal_attention(ptr(x), ptr(x), ptr(x), ptr(i), ptr(i), ptr(x), 1, 1, 32, ps, 1,
                                                 stream())
        assert rc == 1  # CBIS_ERR_INVALID
    rc = K.cbis_fused_paged_causal_attention(ptr(x), ptr(x), ptr(x), ptr(i), ptr(i), ptr(x), 1, 1, 64, 8, 1, stream())
    assert rc == 2  # CBIS_ERR_UNSUPPORTED: the reference kernel needs head_dim 32 too
    sync()


def test_decode_attention_c3_full_size(cbis, oracle, dev):
    """Config 3 at full size: 256 sequences, kv U[128, 2048], 8x32,
    fp32 K/V in a 40,000-page pool with a permuted page table."""
    import torch
    H, P = 8, 40000
    kv, bt = _c3_inputs(oracle)
    n = kv.size
    kp = torch.empty((P, 16, H, 32), dtype=torch.float32, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, s in ((kp, 1), (vp, 2), (q, 3)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), cbis.F32, t.numel(), s, 1.0, stream()))
    pos = kv - 1
    BT, POS = to_dev(bt, dev), to_dev(pos, dev)
    out_split = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
    d = _attn_desc(cbis, n, H, q, kp, vp, P, BT, bt.shape[1], POS, out_split, cbis.F32, max_kv=int(kv.max()))
    need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
    assert need > 0
    ws = torch.empty(need // 4 + 1, dtype=torch.float32, device=dev)
    d.workspace, d.workspace_bytes = ptr(ws), need
    cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
    # the reference-signature entry point (single pass, no workspace) on a
    # [rows, pages_per_seq] row page table
    out_ref_api = torch.empty_like(out_split)
    cbis.check(K.cbis_fused_paged_causal_attention(ptr(q), ptr(kp), ptr(vp), ptr(BT), ptr(POS), ptr(out_ref_api), n, H,
                                                   32, 16, bt.shape[1], stream()))
    sync()
    ref = oracle.paged_attention(q.cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy(), bt, pos, H, 32, 16)
    assert np.abs(out_split.cpu().numpy() - ref).max() < FP32_TOL
    assert np.abs(out_ref_api.cpu().numpy() - ref).max() < FP32_TOL


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_decode_attention_bf16_rows_subset(cbis, oracle, dev, out_dtype):
    """bf16 pools with 64 heads, a row subset (rows list + row->table map),
    kv lengths that end mid-page and a forced small split."""
    import torch
    H, P, S = 64, 3000, 12
    kv = np.array([1, 15, 16, 17, 33, 100, 255, 256, 257, 1000, 2049, 4096], np.int32)
    npages = (kv + 15) // 16
    perm = rng(2).permutation(P).astype(np.int32)
    bt = np.zeros((S, int(npages.max())), np.int32)
    off = 0
    for i in range(S):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    M = 20  # rows; row r belongs to sequence row_bt[r]
    row_bt = rng(3).integers(0, S, M).astype(np.int32)
    pos = np.array([rng(4 + r).integers(0, kv[row_bt[r]]) for r in range(M)], np.int32)
    rows = np.array(sorted(rng(5).choice(M, 15, replace=False)), np.int32)
    kp = torch.empty((P, 16, H, 32), dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((M, H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, s, dt in ((kp, 11, cbis.BF16), (vp, 12, cbis.BF16), (q, 13, cbis.F32)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), dt, t.numel(), s, 1.0, stream()))
    odt = torch.float32 if out_dtype == "f32" else torch.bfloat16
    ref = oracle.paged_attention(q.cpu().numpy()[rows], bits_u16(kp), bits_u16(vp), bt, pos[rows], H, 32, 16,
                                 row_bt=row_bt[rows], kv_dtype=1)
    for split in (0, 64, 1 << 20):
        out = torch.full((M, H * 32), 7.0, dtype=odt, device=dev)
        d = _attn_desc(cbis, len(rows), H, q, kp, vp, P, to_dev(bt, dev), bt.shape[1], to_dev(pos, dev), out,
                       cbis.BF16, out_dtype=cbis.DTYPES[out_dtype], rows=to_dev(rows, dev),
                       row_bt=to_dev(row_bt, dev), max_kv=int(kv.max()), split=split)
        need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
        d.workspace, d.workspace_bytes = ptr(ws), need
        cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
        sync()
        got = out.float().cpu().numpy()
        if out_dtype == "f32":
            assert np.abs(got[rows] - ref).max() < FP32_TOL, split
        else:
            assert row_rel_err(got[rows], ref) < LOWP_TOL, split
        others = np.setdiff1d(np.arange(M), rows)
        assert (got[others] == 7.0).all()  # rows outside the list untouched


def test_decode_attention_closed_forms(cbis, oracle, dev):
    """kv_len = 1 gives v0 exactly; identical keys give the mean of V."""
    import torch
    H, P = 8, 64
    kp = torch.zeros((P, 16, H, 32), dtype=torch.float32, device=dev)
    vp = torch.empty_like(kp)
    K = cbis.kernels()
    cbis.check(K.cbis_fill_normal_fast(ptr(vp), cbis.F32, vp.numel(), 21, 1.0, stream()))
    q = torch.empty((2, H * 32), dtype=torch.float32, device=dev)
    cbis.check(K.cbis_fill_normal_fast(ptr(q), cbis.F32, q.numel(), 22, 1.0, stream()))
    bt = np.array([[5, 9, 2, 0], [7, 1, 3, 4]], np.int32)
    pos = np.array([0, 50], np.int32)   # kv_len 1 and 51 (all keys zero -> equal scores)
    out = torch.empty((2, H * 32), dtype=torch.float32, device=dev)
    d = _attn_desc(cbis, 2, H, q, kp, vp, P, to_dev(bt, dev), 4, to_dev(pos, dev), out, cbis.F32)
    cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
    sync()
    v = vp.cpu().numpy()
    o = out.cpu().numpy().reshape(2, H, 32)
    assert np.array_equal(o[0], v[5, 0])
    keys = [v[bt[1, j // 16], j % 16] for j in range(51)]
    assert np.abs(o[1] - np.mean(keys, axis=0)).max() < 1e-5


def test_decode_attention_max_context(cbis, oracle, dev):
    """Rows at the reference's kMaxSeqLen (kv_len 32768, include/config.hpp)
    and one below, next to a 1-token row, bf16 K/V with 64 heads over a
    permuted pool: the config-5 decode shape against the fp64 oracle."""
    import torch
    H = 64
    kv = np.array([32768, 32767, 1, 32768], np.int32)
    npages = (kv + 15) // 16
    P = int(npages.sum()) + 8
    perm = rng(9).permutation(P).astype(np.int32)
    bt = np.zeros((len(kv), int(npages.max())), np.int32)
    off = 0
    for i in range(len(kv)):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    kp = torch.empty((P, 16, H, 32), dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((len(kv), H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, sd, dt in ((kp, 31, cbis.BF16), (vp, 32, cbis.BF16), (q, 33, cbis.F32)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), dt, t.numel(), sd, 1.0, stream()))
    pos = kv - 1
    out = torch.empty((len(kv), H * 32), dtype=torch.float32, device=dev)
    d = _attn_desc(cbis, len(kv), H, q, kp, vp, P, to_dev(bt, dev), bt.shape[1], to_dev(pos, dev), out,
                   cbis.BF16, max_kv=int(kv.max()))
    need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
    ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
    d.workspace, d.workspace_bytes = ptr(ws), need
    cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
    sync()
    ref = oracle.paged_attention(q.cpu().numpy(), bits_u16(kp), bits_u16(vp), bt, pos, H, 32, 16, kv_dtype=1)
    assert np.abs(out.cpu().numpy() - ref).max() < FP32_TOL


def test_decode_attention_row_order_invariant(cbis, oracle, dev):
    """The row list only orders the work (TransformerRunner passes rows
    longest-first): any order gives bit-identical outputs."""
    import torch
    H, P, n = 16, 2000, 24
    kv = oracle.uniform_int(4, 77, n, 1, 1500)
    npages = (kv + 15) // 16
    perm = rng(6).permutation(P).astype(np.int32)
    bt = np.zeros((n, int(npages.max())), np.int32)
    off = 0
    for i in range(n):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    kp = torch.empty((P, 16, H, 32), dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, sd, dt in ((kp, 41, cbis.BF16), (vp, 42, cbis.BF16), (q, 43, cbis.F32)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), dt, t.numel(), sd, 1.0, stream()))
    outs = []
    for order in (np.arange(n), np.argsort(-kv, kind="stable"), rng(7).permutation(n)):
        out = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
        d = _attn_desc(cbis, n, H, q, kp, vp, P, to_dev(bt, dev), bt.shape[1], to_dev(kv - 1, dev), out, cbis.BF16,
                       rows=to_dev(order.astype(np.int32), dev), max_kv=int(kv.max()))
        need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
        d.workspace, d.workspace_bytes = ptr(ws), need
        cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
        sync()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_empty_calls_are_no_ops(cbis, dev):
    """Zero rows / tiles / tokens: every entry point returns success without
    launching (the reference's forward_step returns {} on an empty batch,
    src/transformer.cpp:47)."""
    K = cbis.kernels()
    d = cbis.GemmDesc()
    d.M, d.N, d.K = 0, 64, 64
    d.x_dtype = d.w_dtype = cbis.BF16
    assert K.cbis_gemm(ctypes.byref(d), None) == 0
    a = cbis.AttnDesc()
    a.n_rows, a.n_heads, a.head_dim, a.page_size = 0, 16, 32, 16
    a.kv_dtype, a.num_pages, a.bt_stride = cbis.BF16, 1, 1
    a.q = a.k_pool = a.v_pool = a.block_table = a.out = a.row_pos = 256  # never dereferenced
    assert K.cbis_paged_attention(ctypes.byref(a), None) == 0
    assert K.cbis_paged_prefill_attention(ctypes.byref(a), 0, None, None) == 0
    assert K.cbis_embed(0, 256, None, None, cbis.F32, None, None, 10, 10, None, None) == 0
    assert K.cbis_layernorm(0, 256, None, 256, None, None, 1e-5, cbis.F32, None, 256, None) == 0
    assert K.cbis_argmax_rows(0, 10, None, 10, None, None) == 0
    cfg = cbis.ModelConfig.make(vocab=512, n_layers=1, max_seq=64)
    w = cbis.ModelWeights.synthetic(cfg, seed=0)
    cache = cbis.PagedKVCache(1, 8, 16, 8, 32, "f32", pages_per_seq=4)
    runner = cbis.TransformerRunner(w, cache, 16)
    assert runner.forward_step([], [], []).size == 0
    assert runner.forward_step_greedy([], [], []) == []


@pytest.mark.parametrize("kvdt,wdt,H", [("f32", "f32", 8), ("f32", "f32", 2), ("f32", "bf16", 8), ("bf16", "bf16", 16),
                                         ("bf16", "f32", 8), ("bf16", "bf16", 4)])
def test_paged_attention_proj_matches_separate(cbis, oracle, dev, kvdt, wdt, H):
    """cbis_paged_attention_proj against cbis_paged_attention (its output
    stored in the projection's X dtype) followed by cbis_gemm with scale-free
    weights, bias and the residual (Y aliasing it): a row subset through
    rows / row_bt, kv lengths 1..768 ending mid-page.  The attention output
    is the same to the bit before the projection (same kernel, same wave
    split); only the projection's summation order differs.  Rows outside the
    list keep their residual."""
    import torch
    D, P, S, M = 32 * H, 700, 6, 12
    kv = np.array([1, 15, 16, 100, 500, 768], np.int32)
    npages = (kv + 15) // 16
    perm = rng(21).permutation(P).astype(np.int32)
    bt = np.zeros((S, int(npages.max())), np.int32)
    off = 0
    for i in range(S):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    row_bt = rng(22).integers(0, S, M).astype(np.int32)
    row_bt[:S] = np.arange(S)  # every length appears
    pos = np.array([kv[row_bt[r]] - 1 if r < S else rng(23 + r).integers(0, kv[row_bt[r]]) for r in range(M)],
                   np.int32)
    rows = np.array(sorted(set(range(S)) | set(rng(24).choice(np.arange(S, M), 3, replace=False).tolist())),
                    np.int32)
    kvt = torch.float32 if kvdt == "f32" else torch.bfloat16
    kp = torch.empty((P, 16, H, 32), dtype=kvt, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((M, D), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, sd in ((kp, 31), (vp, 32), (q, 33)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), cbis.DTYPES[kvdt] if t is not q else cbis.F32, t.numel(), sd, 1.0,
                                           stream()))
    wt = torch.float32 if wdt == "f32" else torch.bfloat16
    W = (torch.randn((D, D), generator=torch.Generator().manual_seed(34)) * 0.05).to(wt).to(dev)
    bias = (torch.randn(D, generator=torch.Generator().manual_seed(35)) * 0.1).to(dev)
    resid = torch.randn((M, D), generator=torch.Generator().manual_seed(36)).to(dev)
    xdt = "f32" if wdt == "f32" else "bf16"
    BT, POS, ROWS, RBT = to_dev(bt, dev), to_dev(pos, dev), to_dev(rows, dev), to_dev(row_bt, dev)
    # separate: attention into X, then the GEMM in place on a residual copy
    attn = torch.zeros((M, D), dtype=torch.float32 if xdt == "f32" else torch.bfloat16, device=dev)
    d = _attn_desc(cbis, len(rows), H, q, kp, vp, P, BT, bt.shape[1], POS, attn, cbis.DTYPES[kvdt],
                   out_dtype=cbis.DTYPES[xdt], rows=ROWS, row_bt=RBT, max_kv=int(kv.max()))
    cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
    y_sep = resid.clone()
    _gemm(cbis, M, D, D, attn, cbis.DTYPES[xdt], W, cbis.DTYPES[wdt], y_sep, cbis.F32, bias=bias, residual=y_sep)
    # fused
    y = resid.clone()
    g = cbis.GemmDesc()
    g.M, g.N, g.K = M, D, D
    g.x_dtype, g.X, g.ldx = cbis.DTYPES[xdt], 0, D
    g.w_dtype, g.W, g.ldw = cbis.DTYPES[wdt], ptr(W), D
    g.bias, g.residual, g.ldr = ptr(bias), ptr(y), D
    g.y_dtype, g.Y, g.ldy = cbis.F32, ptr(y), D
    cbis.check(K.cbis_paged_attention_proj(ctypes.byref(d), ctypes.byref(g), stream()))
    sync()
    got, ref, r0 = y.cpu().numpy(), y_sep.cpu().numpy(), resid.cpu().numpy()
    err = np.abs(got[rows] - ref[rows]).max()
    assert err <= 1e-5 * max(1.0, np.abs(ref[rows]).max()), err
    others = np.setdiff1d(np.arange(M), rows)
    assert np.array_equal(got[others], r0[others])
    # and the attention itself against the oracle (fp32 X only: exact output)
    if xdt == "f32":
        kvb = (lambda t: t.cpu().numpy()) if kvdt == "f32" else bits_u16
        ra = oracle.paged_attention(q.cpu().numpy()[rows], kvb(kp), kvb(vp), bt, pos[rows], H, 32, 16,
                                    row_bt=row_bt[rows], kv_dtype=0 if kvdt == "f32" else 1)
        proj = ra.astype(np.float64) @ W.float().cpu().numpy().T.astype(np.float64) + bias.cpu().numpy() + r0[rows]
        assert np.abs(got[rows] - proj).max() < FP32_TOL


def test_paged_attention_proj_rejects_unsupported(cbis, dev):
    """Widths past one head block or the weight budget, fp8 weights, GELU,
    K/V scatter and a projection of another width are refused before any
    launch (all pointers are dummies that are never dereferenced)."""
    K = cbis.kernels()

    def call(H, kvdt, wdt, **kw):
        a = cbis.AttnDesc()
        a.n_rows, a.n_heads, a.head_dim, a.page_size = 4, H, 32, 16
        a.q_dtype, a.kv_dtype, a.out_dtype = cbis.F32, kvdt, cbis.F32
        a.q = a.k_pool = a.v_pool = a.block_table = a.row_pos = 256
        a.ldq, a.num_pages, a.bt_stride = 32 * H, 16, 4
        g = cbis.GemmDesc()
        g.M, g.N, g.K = 4, kw.get("N", 32 * H), 32 * H
        g.x_dtype, g.w_dtype, g.y_dtype = cbis.F32, wdt, cbis.F32
        g.W = g.Y = 256
        g.ldw = g.ldy = g.ldr = 32 * H
        g.epilogue = kw.get("epi", cbis.EPI_NONE)
        if kw.get("kv"):
            g.k_pool = g.v_pool = 256
        return K.cbis_paged_attention_proj(ctypes.byref(a), ctypes.byref(g), None)

    assert call(64, cbis.BF16, cbis.BF16) != 0          # 2048 wide: many head blocks
    assert call(16, cbis.F32, cbis.F32) != 0            # fp32 K/V: 8 heads per block
    assert call(16, cbis.BF16, cbis.F32) != 0           # 512 fp32 weight columns per thread budget
    assert call(3, cbis.F32, cbis.F32) != 0             # 96: not a multiple of 64
    assert call(8, cbis.F32, cbis.FP8E4M3) != 0         # fp8 weights
    assert call(8, cbis.F32, cbis.F32, epi=cbis.EPI_GELU) != 0
    assert call(8, cbis.F32, cbis.F32, kv=True) != 0
    assert call(8, cbis.F32, cbis.F32, N=128) != 0


def test_decode_attention_rejects_unsupported(cbis):
    d = cbis.AttnDesc()
    d.n_rows, d.n_heads, d.head_dim, d.page_size = 4, 8, 64, 16
    d.q = d.k_pool = d.v_pool = d.block_table = d.out = d.row_pos = 256
    d.num_pages, d.bt_stride = 10, 4
    assert cbis.kernels().cbis_paged_attention(ctypes.byref(d), None) == 2
    d.head_dim = 32
    d.max_kv_len, d.split_tokens = 4096, 64  # needs a workspace
    assert cbis.kernels().cbis_paged_attention(ctypes.byref(d), None) == 3


@pytest.mark.parametrize("n_dec,with_prefill", [(40, True), (40, False), (0, True)])
def test_paged_attention_mixed_matches_two_calls(cbis, dev, n_dec, with_prefill):
    """cbis_paged_attention_mixed (decode rows + prefill tiles, the decode
    split merge folded into the prefill launch) against cbis_paged_attention
    followed by cbis_paged_prefill_attention: bit-identical outputs; with and
    without tiles (the merge then runs on its own) and without decode rows."""
    import torch
    H, cached, n_pf = 64, 37, 100
    kv = rng(11).integers(100, 3000, n_dec).astype(np.int32)
    n_pages = [int(k + 15) // 16 for k in kv] + [(cached + n_pf + 15) // 16]
    P = sum(n_pages) + 8
    perm = rng(12).permutation(P).astype(np.int32)
    width = max(n_pages)
    bt = np.zeros((n_dec + 1, width), np.int32)
    off = 0
    for i, n in enumerate(n_pages):
        bt[i, :n] = perm[off:off + n]
        off += n
    n_rows = n_dec + n_pf
    pos = np.concatenate([kv - 1, cached + np.arange(n_pf)]).astype(np.int32)
    row_bt = np.concatenate([np.arange(n_dec), np.full(n_pf, n_dec)]).astype(np.int32)
    kp = torch.empty((P, 16, H, 32), dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((n_rows, H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, sd, dt in ((kp, 41, cbis.BF16), (vp, 42, cbis.BF16), (q, 43, cbis.F32)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), dt, t.numel(), sd, 1.0, stream()))
    tiles = []
    if with_prefill:
        for r in range(0, n_pf, 64):
            tiles += [n_dec + r, min(64, n_pf - r), n_dec, cached + r]
    T = to_dev(np.array(tiles or [0, 0, 0, 0], np.int32), dev)
    BT, POS, RBT = to_dev(bt, dev), to_dev(pos, dev), to_dev(row_bt, dev)
    ROWS = to_dev(np.arange(max(1, n_dec), dtype=np.int32), dev)
    outs = []
    for mixed in (True, False):
        out = torch.zeros((n_rows, H * 32), dtype=torch.bfloat16, device=dev)
        d = _attn_desc(cbis, n_dec, H, q, kp, vp, P, BT, width, POS, out, cbis.BF16, out_dtype=cbis.BF16, rows=ROWS,
                       row_bt=RBT, max_kv=int(kv.max()) if n_dec else 0)
        need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
        d.workspace, d.workspace_bytes = ptr(ws), need
        d.keep_alive = d.keep_alive + (ws,)
        if n_dec:
            assert need > 0  # the decode rows split: the merge path is exercised
        nt = len(tiles) // 4
        if mixed:
            cbis.check(K.cbis_paged_attention_mixed(ctypes.byref(d), nt, ptr(T), stream()), "mixed")
        else:
            if n_dec:
                cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()), "decode")
            cbis.check(K.cbis_paged_prefill_attention(ctypes.byref(d), nt, ptr(T), stream()), "prefill")
        sync()
        outs.append(out.view(torch.int16).cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    written = np.zeros(n_rows, bool)
    written[:n_dec] = True
    if with_prefill:
        written[n_dec:] = True
    assert (outs[0][written] != 0).any(axis=1).all()


@pytest.mark.parametrize("cached,n_rows,tile", [(0, 100, 64), (37, 64, 64), (512, 512, 64), (37, 70, 32),
                                                (5, 9, 64)])
def test_prefill_attention_mfma(cbis, oracle, dev, cached, n_rows, tile):
    """A chunk of n_rows consecutive positions after `cached` cached tokens
    (config 4's chunks are (0, 512) and (512, 512)), in tiles of `tile` rows
    (the runner's 64, ragged last tiles; 32-row tiles are valid too)."""
    import torch
    H, P = 64, 200
    total = cached + n_rows
    npages = (total + 15) // 16
    bt = rng(7).permutation(P)[:npages].astype(np.int32)[None, :]
    kp = torch.empty((P, 16, H, 32), dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((n_rows, H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, s, dt in ((kp, 31, cbis.BF16), (vp, 32, cbis.BF16), (q, 33, cbis.F32)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), dt, t.numel(), s, 1.0, stream()))
    pos = (cached + np.arange(n_rows)).astype(np.int32)
    tiles, tiles12 = [], []
    for r in range(0, n_rows, tile):
        nv = min(tile, n_rows - r)
        tiles += [r, nv, 0, cached + r]
        # the 12-int form: the tile's first 8 page ids, page min(16 k, kv_end - 1) / 16
        tiles12 += [r, nv, 0, cached + r] + [int(bt[0, min(16 * k, cached + r + nv - 1) // 16]) for k in range(8)]
    T = to_dev(np.array(tiles, np.int32), dev)
    out = torch.empty((n_rows, H * 32), dtype=torch.bfloat16, device=dev)
    d = _attn_desc(cbis, n_rows, H, q, kp, vp, P, to_dev(bt, dev), bt.shape[1], None, out, cbis.BF16,
                   out_dtype=cbis.BF16)
    cbis.check(K.cbis_paged_prefill_attention(ctypes.byref(d), len(tiles) // 4, ptr(T), stream()))
    # The same tiles with their first pages in the descriptor: the same loads, bit for bit.
    T12 = to_dev(np.array(tiles12, np.int32), dev)
    out12 = torch.empty_like(out)
    d12 = _attn_desc(cbis, n_rows, H, q, kp, vp, P, to_dev(bt, dev), bt.shape[1], None, out12, cbis.BF16,
                     out_dtype=cbis.BF16)
    d12.tile_pages = 8
    cbis.check(K.cbis_paged_prefill_attention(ctypes.byref(d12), len(tiles12) // 12, ptr(T12), stream()))
    d12.tile_pages = 4
    assert K.cbis_paged_prefill_attention(ctypes.byref(d12), len(tiles12) // 12, ptr(T12), stream()) != 0
    sync()
    assert torch.equal(out12.view(torch.int16), out.view(torch.int16))
    ref = oracle.paged_attention(q.cpu().numpy(), bits_u16(kp), bits_u16(vp), np.repeat(bt, n_rows, 0), pos, H, 32,
                                 16, kv_dtype=1)
    got = out.float().cpu().numpy()
    # The bf16 parity metric: per row, ||d||_inf / ||ref||_inf over the
    # row's H * head_dim outputs.  Q and P are rounded to bf16 for the MFMAs.
    err_row = row_rel_err(got, ref)
    err_head = row_rel_err(got.reshape(n_rows * H, 32), ref.reshape(n_rows * H, 32))
    print(f"prefill cached={cached} rows={n_rows} tile={tile}: per-row rel {err_row:.3e}, "
          f"per-(row, head) rel {err_head:.3e}", flush=True)
    assert err_row < LOWP_TOL
    assert err_head < LOWP_TOL * 2   # stricter slicing: each head against its own maximum
    assert np.abs(got - ref).mean() < 2e-3


def _lazy_raises(scores, qpos, kv_end, waves=2, thr=8.0):
    """The prefill kernel's lazy softmax reference, simulated per query row:
    a head's waves take its 32-key blocks round-robin (wave w: blocks w,
    w + waves, ...), m starts at -inf, a block's first unmasked key sets m,
    and a finite m is raised only when the block's maximum over the row's
    visible keys exceeds it by more than `thr` (log2 units).  scores
    [rows, keys] in log2 units.  Returns, per row, how many finite-m raises
    its waves made."""
    n_rows = scores.shape[0]
    out = np.zeros(n_rows, np.int64)
    nblk = (kv_end + 31) // 32
    for r in range(n_rows):
        vis = min(int(qpos[r]) + 1, kv_end)
        for w in range(waves):
            m = -np.inf
            for b in range(w, nblk, waves):
                lo, hi = 32 * b, min(32 * b + 32, vis)
                if hi <= lo:
                    continue
                smax = scores[r, lo:hi].max()
                if m == -np.inf:
                    m = smax
                elif smax - m > thr:
                    m = smax
                    out[r] += 1
    return out


@pytest.mark.parametrize("mode", ["planted", "q_scaled"])
def test_prefill_attention_lazy_rescale(cbis, oracle, dev, mode):
    """Inputs whose later key blocks dominate, so a wave's finite softmax
    reference m is raised mid-sequence (o and the row sums rescaled by
    2^(m_old - m_new), the block's scores shifted, -m reloaded) -- a path
    N(0, 1) inputs never take (their scaled scores spread ~1.4 log2 units).

    planted: every query row of a head is the same vector u and key j is
    a_j u / |u|^2 / qscale, so its score is a_j log2 units: ~400 flat keys
    (a ~ N(0, 0.3)), then one spike key per wave at +9.5, past the 8-unit
    threshold.  The flat keys then still carry ~20% of the softmax mass
    after the rescale, so a wrong correction factor moves the output by
    several percent.  q_scaled: Q ~ N(0, 16) (scores spread ~5.8 log2
    units), K / V ~ N(0, 1).  Both: 100 query rows after 380 cached keys,
    tiles of 64 (the second ragged), blocks straddling the causal diagonal.
    A host simulation of the kernel's block order asserts the raises happen.
    The output is checked against the fp64 oracle with the per-row metric,
    and, tighter, against the oracle given the kernel's bf16-rounded Q (the
    scaled Q is an MFMA operand; at scores of tens of log2 units its
    rounding alone moves the softmax weights by a few percent, which is not
    what this test is about)."""
    import torch
    H, P, cached, n_rows, HD = 64, 64, 380, 100, 32
    qscale = np.log2(np.e) / np.sqrt(HD)
    total = cached + n_rows
    npages = (total + 15) // 16
    bt = rng(71).permutation(P)[:npages].astype(np.int32)[None, :]
    g = rng(72)
    v = g.standard_normal((total, H, HD)).astype(np.float32)
    if mode == "planted":
        u = g.standard_normal((H, HD))
        a = g.normal(0.0, 0.3, total)
        spikes = [405, 440]  # key blocks 12 (wave 0) and 13 (wave 1)
        a[spikes] = 9.5
        k = (a[:, None, None] * u[None] / (u * u).sum(-1)[None, :, None] / qscale).astype(np.float32)
        qh = np.broadcast_to(u[None], (n_rows, H, HD)).astype(np.float32).reshape(n_rows, H * HD)
    else:
        k = g.standard_normal((total, H, HD)).astype(np.float32)
        qh = (4.0 * g.standard_normal((n_rows, H * HD))).astype(np.float32)
    kd, kvals = bf16_dev(k, dev)
    vd, _ = bf16_dev(v, dev)
    kp = torch.zeros((P, 16, H, HD), dtype=torch.bfloat16, device=dev)
    vp = torch.zeros_like(kp)
    for j in range(npages):
        n = min(16, total - 16 * j)
        kp[int(bt[0, j]), :n] = kd[16 * j: 16 * j + n]
        vp[int(bt[0, j]), :n] = vd[16 * j: 16 * j + n]
    q = to_dev(qh, dev)
    pos = (cached + np.arange(n_rows)).astype(np.int32)
    tiles = []
    for r in range(0, n_rows, 64):
        tiles += [r, min(64, n_rows - r), 0, cached + r]
    T = to_dev(np.array(tiles, np.int32), dev)
    out = torch.empty((n_rows, H * HD), dtype=torch.bfloat16, device=dev)
    d = _attn_desc(cbis, n_rows, H, q, kp, vp, P, to_dev(bt, dev), bt.shape[1], None, out, cbis.BF16,
                   out_dtype=cbis.BF16)
    cbis.check(cbis.kernels().cbis_paged_prefill_attention(ctypes.byref(d), len(tiles) // 4, ptr(T), stream()))
    sync()
    # The raises the kernel's block order makes, from the bf16 operands it
    # reads (Q rounded after the scale, as the kernel does).
    qb = torch.from_numpy(qh * np.float32(qscale)).to(torch.bfloat16).float().numpy().reshape(n_rows, H, HD)
    raises = np.zeros(n_rows, np.int64)
    for h in range(H):
        s = qb[:, h, :].astype(np.float64) @ kvals[:, h, :].astype(np.float64).T
        raises += _lazy_raises(s, pos, total)
    rows_raised = int((raises > 0).sum())
    ref = oracle.paged_attention(qh, bits_u16(kp), bits_u16(vp), np.repeat(bt, n_rows, 0), pos, H, HD, 16,
                                 kv_dtype=1)
    got = out.float().cpu().numpy()
    err_row = row_rel_err(got, ref)
    err_head = row_rel_err(got.reshape(n_rows * H, HD), ref.reshape(n_rows * H, HD))
    q_rounded = (qb.reshape(n_rows, H * HD) / np.float32(qscale)).astype(np.float32)
    ref_qb = oracle.paged_attention(q_rounded, bits_u16(kp), bits_u16(vp), np.repeat(bt, n_rows, 0), pos, H, HD,
                                    16, kv_dtype=1)
    err_qb = row_rel_err(got, ref_qb)
    print(f"prefill lazy rescale ({mode}): {int(raises.sum())} finite-m raises over {rows_raised} rows; "
          f"per-row rel {err_row:.3e}, per-(row, head) rel {err_head:.3e}; against bf16-Q oracle {err_qb:.3e}",
          flush=True)
    assert err_qb < 1e-2
    if mode == "planted":
        # every row past a spike raises in the wave that holds it, every head
        assert (raises[pos >= 405] >= H).all() and (raises[pos >= 440] >= 2 * H).all()
    else:
        assert rows_raised >= n_rows // 2
    assert err_row < LOWP_TOL
    assert err_head < LOWP_TOL * 2


@pytest.mark.parametrize("kv_dtype,H", [("f32", 12), ("f32", 4), ("bf16", 24), ("bf16", 8)])
def test_decode_attention_any_head_count(cbis, oracle, dev, kv_dtype, H):
    """Head counts that do not fill the last 1 KiB head block (8 fp32 or 16
    bf16 heads), as the reference's grid(total_rows, n_heads) allows
    (kernels/attention.cu:113-127): through the reference-signature entry
    point (fp32) and the split-KV entry point with partials and merge."""
    import torch
    S, P = 10, 900
    kv = np.array([1, 16, 17, 40, 333, 700, 1200, 64, 5, 999], np.int32)
    npages = (kv + 15) // 16
    perm = rng(21).permutation(P).astype(np.int32)
    bt = np.zeros((S, int(npages.max())), np.int32)
    off = 0
    for i in range(S):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    tdt, cdt, kd = (torch.float32, cbis.F32, 0) if kv_dtype == "f32" else (torch.bfloat16, cbis.BF16, 1)
    kp = torch.empty((P, 16, H, 32), dtype=tdt, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((S, H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, sd, dt in ((kp, 51, cdt), (vp, 52, cdt), (q, 53, cbis.F32)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), dt, t.numel(), sd, 1.0, stream()))
    pos = kv - 1
    BT, POS = to_dev(bt, dev), to_dev(pos, dev)
    host = (lambda t: t.cpu().numpy()) if kd == 0 else bits_u16
    ref = oracle.paged_attention(q.cpu().numpy(), host(kp), host(vp), bt, pos, H, 32, 16, kv_dtype=kd)
    outs = []
    if kd == 0:
        o = torch.full((S, H * 32), 7.0, dtype=torch.float32, device=dev)
        cbis.check(K.cbis_fused_paged_causal_attention(ptr(q), ptr(kp), ptr(vp), ptr(BT), ptr(POS), ptr(o), S, H, 32,
                                                       16, bt.shape[1], stream()))
        outs.append(o)
    for split in (64, 0):
        o = torch.full((S, H * 32), 7.0, dtype=torch.float32, device=dev)
        d = _attn_desc(cbis, S, H, q, kp, vp, P, BT, bt.shape[1], POS, o, cdt, max_kv=int(kv.max()), split=split)
        need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
        d.workspace, d.workspace_bytes = ptr(ws), need
        d.keep_alive = d.keep_alive + (ws,)
        if split == 64:
            assert need == S * ((int(kv.max()) + 63) // 64) * H * 36 * 4
        cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
        sync()
        outs.append(o)
    sync()
    for o in outs:
        got = o.cpu().numpy()
        if kd == 0:
            assert np.abs(got - ref).max() < FP32_TOL
        else:
            assert row_rel_err(got, ref) < LOWP_TOL
        assert (got != 7.0).all()   # every head of every row written, nothing past the last head


@pytest.mark.parametrize("n_heads", [8, 12])
def test_scatter_kv_to_cache_reference_signature(cbis, oracle, dev, n_heads):
    """cbis_scatter_kv_to_cache (include/attention.hpp:8-12) bit-exact
    against the oracle's restatement of kernels/attention.cu:7-19: rows go
    to permuted (page, slot) pairs, every other slot keeps its bytes."""
    import torch
    D, P, M = n_heads * 32, 37, 150
    slots = rng(31).permutation(P * 16)[:M]
    wpage, woff = (slots // 16).astype(np.int32), (slots % 16).astype(np.int32)
    kv_rows = oracle.normal(31, 1, 2 * M * D).reshape(2, M, D)
    k_host = oracle.normal(31, 2, P * 16 * D).reshape(P, 16, n_heads, 32)
    v_host = oracle.normal(31, 3, P * 16 * D).reshape(P, 16, n_heads, 32)
    kp, vp = to_dev(k_host, dev), to_dev(v_host, dev)
    Kr, Vr, WP, WO = to_dev(kv_rows[0], dev), to_dev(kv_rows[1], dev), to_dev(wpage, dev), to_dev(woff, dev)
    K = cbis.kernels()
    cbis.check(K.cbis_scatter_kv_to_cache(ptr(Kr), ptr(Vr), ptr(kp), ptr(vp), ptr(WP), ptr(WO), M, D, 16, n_heads, 32,
                                          stream()))
    sync()
    ek, ev = k_host.copy(), v_host.copy()
    oracle.scatter_kv(kv_rows[0], kv_rows[1], ek, ev, wpage, woff, 16)
    assert np.array_equal(kp.cpu().numpy().view(np.uint32), ek.view(np.uint32))
    assert np.array_equal(vp.cpu().numpy().view(np.uint32), ev.view(np.uint32))
    assert K.cbis_scatter_kv_to_cache(ptr(Kr), ptr(Vr), ptr(kp), ptr(vp), ptr(WP), ptr(WO), M, D + 1, 16, n_heads, 32,
                                      stream()) == 1


# --------------------------------------------------------------------------
# lm_head fused with the greedy argmax and top-2 margin (cbis_gemm_argmax)
# --------------------------------------------------------------------------

def _top2_np(logits):
    """First index of each row's maximum and max minus the largest value at
    any other index, in fp32 (the margin definition of cbis_gemm_argmax)."""
    lg = np.asarray(logits, np.float32)
    idx = lg.argmax(axis=1)
    rest = lg.copy()
    rest[np.arange(len(lg)), idx] = -np.inf
    m1 = lg[np.arange(len(lg)), idx]
    return idx, (m1 - rest.max(axis=1)).astype(np.float32)


@pytest.mark.parametrize("M,N,K,wdt", [
    (7, 32000, 2048, "bf16"),     # skinny kernel, 2000 partials per row
    (16, 32000, 2048, "fp8"),     # skinny, fp8 codes with channel scales (config 5's lm_head)
    (8, 512, 256, "f32"),         # skinny fp32 (config 1's decode steps)
    (1216, 32000, 2048, "bf16"),  # wave-specialised 160 x 256 (config 4's lm_head)
    (300, 32000, 512, "bf16"),    # wave-specialised, ragged last row tile
    (100, 1000, 256, "bf16"),     # small grid: logits stored in Y, then reduced
    (100, 512, 256, "f32"),       # fp32 at M > 64 (config 1's prefill): stored, then reduced
    (200, 1000, 512, "fp8"),      # fp8 at M > 64: stored, then reduced
    (600, 20007, 512, "bf16"),    # wave-specialised, last column tile partial (the column-test epilogue)
    (600, 20480, 512, "bf16-nobias"),  # wave-specialised, no scale or bias (the plain epilogue)
])
def test_gemm_argmax_matches_logits(cbis, oracle, dev, M, N, K, wdt):
    """Tokens and margins of the fused greedy lm_head equal, bit for bit,
    orc_argmax_rows and the top-2 margin of the logits cbis_gemm writes for
    the same descriptor; columns 37 and N - 5 are made equal and the largest
    in rows 0..3 (a tie across column tiles: the lower index wins, margin 0)."""
    import torch
    K_ = cbis.kernels()
    w = oracle.normal(71, 2, N * K, 0.02).reshape(N, K)
    x = oracle.normal(71, 1, M * K).reshape(M, K)
    w[N - 5] = w[37]
    x[:4] = np.abs(x[:4])
    w[37] = np.abs(w[37]) + 0.05
    w[N - 5] = w[37]
    b = oracle.normal(71, 3, N, 0.02)
    b[N - 5] = b[37]
    if wdt == "f32":
        X, W = to_dev(x, dev), to_dev(w, dev)
        xdt, wd, S = cbis.F32, cbis.F32, None
    elif wdt.startswith("bf16"):
        (X, _), (W, _) = bf16_dev(x, dev), bf16_dev(w, dev)
        xdt, wd, S = cbis.BF16, cbis.BF16, None
    else:
        codes, sc = oracle.quantize_e4m3_rows(w)
        sc[N - 5] = sc[37]
        codes[N - 5] = codes[37]
        (X, _), W, S = bf16_dev(x, dev), to_dev(codes, dev), to_dev(sc, dev)
        xdt, wd = cbis.BF16, cbis.FP8E4M3
    B = None if wdt == "bf16-nobias" else to_dev(b, dev)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    d = cbis.GemmDesc()
    d.M, d.N, d.K = M, N, K
    d.x_dtype, d.X, d.ldx = xdt, ptr(X), K
    d.w_dtype, d.W, d.ldw = wd, ptr(W), K
    d.w_scale, d.bias = ptr(S), ptr(B)
    d.y_dtype, d.Y, d.ldy = cbis.F32, ptr(Y), N
    # the logits as cbis_gemm writes them with its split-K workspace, which
    # the greedy call's fallback (paths that store logits) is given as well
    gneed = K_.cbis_gemm_workspace_size(ctypes.byref(d))
    gws = torch.empty(max(1, gneed // 4), dtype=torch.float32, device=dev)
    d.workspace, d.workspace_bytes = ptr(gws), gneed
    cbis.check(K_.cbis_gemm(ctypes.byref(d), stream()), "cbis_gemm")
    sync()
    d.workspace, d.workspace_bytes = None, 0
    logits = Y.cpu().numpy()
    # greedy call: Y poisoned first, so a path that reduces in its epilogue
    # must not depend on it (and one that stores the logits rewrites it)
    Y.fill_(float("nan"))
    need = K_.cbis_gemm_argmax_workspace_size(ctypes.byref(d))
    ws = torch.empty(max(4, need // 4), dtype=torch.float32, device=dev)
    nxt = torch.full((M,), -1, dtype=torch.int32, device=dev)
    mar = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
    cbis.check(K_.cbis_gemm_argmax(ctypes.byref(d), ptr(nxt), ptr(mar), ptr(ws), need, stream()), "cbis_gemm_argmax")
    sync()
    idx, margin = _top2_np(logits)
    assert np.array_equal(nxt.cpu().numpy(), oracle.argmax_rows(logits))
    assert np.array_equal(nxt.cpu().numpy(), idx)
    assert np.array_equal(mar.cpu().numpy().view(np.uint32), margin.view(np.uint32))
    assert (idx[:4] == 37).all() and (margin[:4] == 0).all()
    if need >= 16:
        assert K_.cbis_gemm_argmax(ctypes.byref(d), ptr(nxt), ptr(mar), ptr(ws), need - 16, stream()) == 3


@pytest.mark.parametrize("M,N,K,wdt", [
    (7, 32000, 2048, "bf16"),     # skinny kernel
    (16, 4000, 512, "fp8"),       # skinny, fp8 codes with channel scales
    (8, 512, 256, "f32"),         # skinny fp32
    (300, 32000, 512, "bf16"),    # wave-specialised (greedy epilogue)
    (100, 1000, 256, "bf16"),     # small grid: logits stored, then reduced
    (100, 512, 256, "f32"),       # fp32 at M > 64: stored, then reduced
])
@pytest.mark.parametrize("nan_col", ["first", "middle"])
def test_argmax_nan_rule(cbis, oracle, dev, M, N, K, wdt, nan_col):
    """A NaN logit (planted through the bias, so every row has it in the same
    column) follows the reference's scan (src/bench_batching.cpp:66-73, whose
    first value is never displaced since no comparison with NaN succeeds): at
    column 0 the token is 0 (margin +inf); elsewhere it never wins and the
    margin is the top two of the other columns.  cbis_gemm_argmax on every
    path, and cbis_argmax_rows over the stored logits, against
    orc_argmax_rows."""
    import torch
    K_ = cbis.kernels()
    w = oracle.normal(73, 2, N * K, 0.02).reshape(N, K)
    x = oracle.normal(73, 1, M * K).reshape(M, K)
    b = oracle.normal(73, 3, N, 0.02)
    col = 0 if nan_col == "first" else N // 2 + 3
    b[col] = np.nan
    if wdt == "f32":
        X, W, xdt, wd, S = to_dev(x, dev), to_dev(w, dev), cbis.F32, cbis.F32, None
    elif wdt == "bf16":
        (X, _), (W, _) = bf16_dev(x, dev), bf16_dev(w, dev)
        xdt, wd, S = cbis.BF16, cbis.BF16, None
    else:
        codes, sc = oracle.quantize_e4m3_rows(w)
        (X, _), W, S = bf16_dev(x, dev), to_dev(codes, dev), to_dev(sc, dev)
        xdt, wd = cbis.BF16, cbis.FP8E4M3
    B = to_dev(b, dev)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    d = cbis.GemmDesc()
    d.M, d.N, d.K = M, N, K
    d.x_dtype, d.X, d.ldx = xdt, ptr(X), K
    d.w_dtype, d.W, d.ldw = wd, ptr(W), K
    d.w_scale, d.bias = ptr(S), ptr(B)
    d.y_dtype, d.Y, d.ldy = cbis.F32, ptr(Y), N
    gneed = K_.cbis_gemm_workspace_size(ctypes.byref(d))
    gws = torch.empty(max(1, gneed // 4), dtype=torch.float32, device=dev)
    d.workspace, d.workspace_bytes = ptr(gws), gneed
    cbis.check(K_.cbis_gemm(ctypes.byref(d), stream()), "cbis_gemm")
    sync()
    d.workspace, d.workspace_bytes = None, 0
    logits = Y.cpu().numpy()
    assert np.isnan(logits[:, col]).all() and not np.isnan(np.delete(logits, col, axis=1)).any()
    want = oracle.argmax_rows(logits)
    rows = torch.full((M,), -1, dtype=torch.int32, device=dev)
    cbis.check(K_.cbis_argmax_rows(M, N, ptr(Y), N, ptr(rows), stream()), "cbis_argmax_rows")
    need = K_.cbis_gemm_argmax_workspace_size(ctypes.byref(d))
    ws = torch.empty(max(4, need // 4), dtype=torch.float32, device=dev)
    nxt = torch.full((M,), -1, dtype=torch.int32, device=dev)
    mar = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
    cbis.check(K_.cbis_gemm_argmax(ctypes.byref(d), ptr(nxt), ptr(mar), ptr(ws), need, stream()), "cbis_gemm_argmax")
    sync()
    assert np.array_equal(rows.cpu().numpy(), want)
    assert np.array_equal(nxt.cpu().numpy(), want)
    if nan_col == "first":
        assert (want == 0).all() and np.isposinf(mar.cpu().numpy()).all()
    else:
        rest = logits.copy()
        rest[:, col] = -np.inf
        idx, margin = _top2_np(rest)
        assert np.array_equal(want, idx)
        assert np.array_equal(mar.cpu().numpy().view(np.uint32), margin.view(np.uint32))
