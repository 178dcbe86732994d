"""Projection GEMM parity (y = x W^T) against a plain PyTorch reference.

f16: compared with the f32-accumulated product rounded to half, within one
half ulp plus 1e-3 (the reference's rule, neural.rs:466-480).  f32: compared
with an f64 product, relative to the norm of the terms.  SwiGLU: compared with
the reference's half rounding steps, and with the unfused kernels.
"""
import pytest
import torch

gpu = pytest.mark.gpu


@pytest.fixture(scope="module")
def clef():
    import clef_hip
    clef_hip.lib()
    return clef_hip


def _inputs(seed, M, N, K, dtype):
    import workloads
    return workloads.gemm_inputs(seed, M, N, K, dtype=dtype)


def _check_f16(y, x, w):
    ref = (x.float() @ w.float().T)
    exp = ref.half().float()
    err = (y.float() - exp).abs()
    tol = 1e-3 + exp.abs() * 2.0 ** -10
    assert (err <= tol).all(), f"max err {err.max().item():.3e}"


def _check_f32(y, x, w):
    ref = x.double() @ w.double().T
    scale = x.double().abs() @ w.double().abs().T
    err = (y.double() - ref).abs()
    assert (err <= 1e-5 * scale + 1e-6).all(), f"max rel err {(err / (scale + 1e-30)).max().item():.3e}"


SHAPES = [(1, 1, 1), (17, 73, 65), (139, 129, 128), (17, 73, 4096), (513, 137, 65), (1025, 257, 128),
          (4096, 3000, 256)]  # the last: 192-wide tiles, ragged last column


@gpu
@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_gemm_reference_shapes(clef, M, N, K, dtype):
    """neural.rs:439-480 shapes, including ragged tiles and unaligned K."""
    x, w = _inputs(7, M, N, K, dtype)
    y = clef.gemm(x, w)
    (_check_f16 if dtype == torch.float16 else _check_f32)(y, x, w)


@gpu
@pytest.mark.parametrize("N", [8192, 2048, 6144, 12352, 9216])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_gemm_projection_shapes(clef, N, dtype):
    """M = 2048 tokens, K = 2048 hidden; x ~ N(0,1), W ~ N(0,0.02), seed 1."""
    x, w = _inputs(1, 2048, N, 2048, dtype)
    y = clef.gemm(x, w)
    (_check_f16 if dtype == torch.float16 else _check_f32)(y, x, w)


@gpu
@pytest.mark.parametrize("M,N,K", [(2100, 12300, 128), (2100, 12300, 2048), (2048, 9216, 2048), (4096, 12288, 192),
                                   (2100, 2100, 256),  # 289 tiles of 128 x 128
                                   # 256 x 128 tiles on four waves: one whole round, and
                                   # ragged rows and columns
                                   (4096, 2048, 512), (4000, 1900, 320)])
def test_gemm_persistent_launches(clef, M, N, K):
    """More tiles than CUs: one work-group per CU runs several tiles, the
    next tile's first stages requested during the current one's last.
    Ragged rows and columns, two K stages, a partial last round, 192-wide
    tiles, 128 x 128 tiles (three-slot rings); the f32 output (one tile per
    work-group) must agree bit for bit once rounded."""
    x, w = _inputs(9, M, N, K, torch.float16)
    y = clef.gemm(x, w)
    _check_f16(y, x, w)
    assert torch.equal(clef.gemm(x, w, out_dtype=torch.float32).half(), y)


@gpu
@pytest.mark.parametrize("M,N,K", [(2100, 6150, 128), (2048, 6144, 2048)])
def test_swiglu_persistent_launches(clef, M, N, K):
    gen = torch.Generator(device="cuda").manual_seed(15)
    x = torch.randn((M, K), generator=gen, device="cuda").half()
    wg = (torch.randn((N, K), generator=gen, device="cuda") * 0.05).half()
    wu = (torch.randn((N, K), generator=gen, device="cuda") * 0.05).half()
    y = clef.gemm_swiglu(x, wg, wu)
    assert torch.equal(y, clef.silu_mul(clef.gemm(x, wg), clef.gemm(x, wu)))


@gpu
@pytest.mark.parametrize("M,N,K", [(4096, 2048, 4096), (4096, 2048, 6144), (20, 16, 8), (300, 203, 128),
                                   (4096, 3000, 256),
                                   # residual tiles read during the last eight K stages: full and
                                   # partial tiles in one launch, exactly eight stages, an odd row
                                   # pitch (no vector access), 128 x 128 tiles
                                   (1000, 2000, 1024), (768, 2048, 512), (600, 2001, 1024),
                                   (256, 1024, 768)])
def test_gemm_residual_epilogue(clef, M, N, K):
    x, w = _inputs(3, M, N, K, torch.float16)
    h = torch.randn((M, N), device="cuda")
    h0 = h.clone()
    clef.gemm(x, w, residual=h, out_dtype=torch.float16)
    prod = (x.float() @ w.float().T).half().float()
    exp = h0 + prod
    err = (h - exp).abs()  # one half ulp of the product, plus the f32 add
    assert (err <= 1e-3 + prod.abs() * 2.0 ** -10 + exp.abs() * 2.0 ** -23).all(), \
        f"max err {err.max().item():.3e}"


@gpu
@pytest.mark.parametrize("M,N,K", [(512, 256, 256), (300, 203, 128), (1024, 1024, 1024)])
def test_gemm_residual_epilogue_unrounded(clef, M, N, K):
    """Residual add of the f32 accumulator itself (no half rounding), aligned
    and ragged rows, and residual tiles read during the last K stages."""
    x, w = _inputs(8, M, N, K, torch.float16)
    h = torch.randn((M, N), device="cuda")
    h0 = h.clone()
    clef.gemm(x, w, residual=h, out_dtype=torch.float32)
    prod = x.double() @ w.double().T
    scale = x.double().abs() @ w.double().abs().T
    err = (h.double() - (h0.double() + prod)).abs()
    assert (err <= 1e-5 * scale + 2e-6 * (h0.double().abs() + 1)).all(), f"max err {err.max().item():.3e}"


@gpu
def test_gemm_f16_output_from_f32_accumulator_rounds_once(clef):
    x, w = _inputs(4, 300, 200, 512, torch.float16)
    y32 = clef.gemm(x, w, out_dtype=torch.float32)
    y16 = clef.gemm(x, w)
    assert torch.equal(y32.half(), y16)


@gpu
@pytest.mark.parametrize("M,N,K", [(2048, 6144, 2048), (600, 6144, 2048), (20, 32, 16), (513, 137, 64)])
def test_swiglu_matches_half_rounding_steps_and_unfused_kernels(clef, M, N, K):
    import workloads
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((M, K), generator=gen, device="cuda").half()
    wg = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    wu = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    y = clef.gemm_swiglu(x, wg, wu)
    g16, u16 = clef.gemm(x, wg), clef.gemm(x, wu)
    # the reference's rule: the fused kernel equals the unfused kernels
    assert torch.equal(y, clef.silu_mul(g16, u16))
    # the half-rounding steps with an exactly rounded SiLU: the hardware SiLU
    # moves the rounded silu by one ulp in rare cases, which the product
    # carries to at most two ulps of the output
    g, u = g16.float(), u16.float()
    s = (g / (1.0 + torch.exp(-g))).half().float()
    unfused = (s * u).half()
    diff = (y.float() - unfused.float()).abs()
    ulp = unfused.float().abs().clamp(min=2.0 ** -14) * 2.0 ** -10
    assert (diff <= 2 * ulp).all()
    assert (diff == 0).float().mean() > 0.999
    gr = (x.float() @ wg.float().T).half().float()
    ur = (x.float() @ wu.float().T).half().float()
    ref = ((gr / (1 + torch.exp(-gr))).half().float() * ur).half().float()
    err = (y.float() - ref).abs()
    assert (err <= 1e-3 + ref.abs() * 2.0 ** -9).all(), f"max err {err.max().item():.3e}"


@gpu
def test_swiglu_f32(clef):
    gen = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn((333, 256), generator=gen, device="cuda")
    wg = torch.randn((500, 256), generator=gen, device="cuda") * 0.05
    wu = torch.randn((500, 256), generator=gen, device="cuda") * 0.05
    y = clef.gemm_swiglu(x, wg, wu)
    g = x.double() @ wg.double().T
    ref = torch.nn.functional.silu(g) * (x.double() @ wu.double().T)
    assert (y.double() - ref).abs().max().item() < 1e-4


@gpu
def test_swiglu_f32_projection_shape(clef):
    """The f32 SwiGLU the bench times: M = K = 2048, N = 6144 gate and up,
    x ~ N(0,1), W ~ N(0,0.02) (seeds 1 and 2), against an f64 product; the
    bound carries each projection's f32 accumulation error (relative to its
    terms' magnitudes) through silu(g) u."""
    x, wg = _inputs(1, 2048, 6144, 2048, torch.float32)
    _, wu = _inputs(2, 2048, 6144, 2048, torch.float32)
    y = clef.gemm_swiglu(x, wg, wu).double()
    xd = x.double()
    g, u = xd @ wg.double().T, xd @ wu.double().T
    sg, su = xd.abs() @ wg.double().abs().T, xd.abs() @ wu.double().abs().T
    sil = torch.nn.functional.silu(g)
    ref = sil * u
    tol = 1e-5 * (1.1 * sg * u.abs() + sil.abs() * su) + 2e-6 * ref.abs() + 1e-7
    err = (y - ref).abs()
    assert (err <= tol).all(), f"max err {err.max().item():.3e}, worst ratio {(err / tol).max().item():.2f}"


@gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_silu_mul_matches_the_formula(clef, dt):
    """clef_silu_mul: f32 as silu(g) * u; f16 with the SwiGLU's half roundings,
    the SiLU within one f16 ulp of the exactly rounded one."""
    gen = torch.Generator(device="cuda").manual_seed(12)
    g = (4 * torch.randn(100_003, generator=gen, device="cuda")).to(dt)
    u = torch.randn(100_003, generator=gen, device="cuda").to(dt)
    y = clef.silu_mul(g, u).float()
    gf, uf = g.float(), u.float()
    if dt == torch.float32:
        torch.testing.assert_close(y, gf / (1 + torch.exp(-gf)) * uf, rtol=1e-6, atol=1e-7)
    else:
        ref = ((gf / (1 + torch.exp(-gf))).half().float() * uf).half().float()
        ulp = ref.abs().clamp(min=2.0 ** -14) * 2.0 ** -10
        assert ((y - ref).abs() <= 2 * ulp).all()
        assert (y == ref).float().mean() > 0.999


def test_silu_mul_rejects_bad_arguments(clef):
    """Validation before any launch (no GPU needed)."""
    assert clef.lib().clef_silu_mul(None, None, None, 16, 1, None) < 0
    assert clef.lib().clef_silu_mul(1, 1, 1, 0, 1, None) < 0
    assert clef.lib().clef_silu_mul(1, 1, 1, 16, 7, None) < 0
