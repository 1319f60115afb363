"""Projections vs the oracle: gemv_proj_bf16, gemv_proj_bf162float and
batch_gemv_proj_bf16 through the C ABI.

The reference's own cases (tests/test_gemv_proj_bf16.cu:48-56,
tests/test_gemv_proj_bf162float.cu:45-53, tests/test_batch_gemv_proj_bf16.cu:
108-111) are checked at their bar (8e-2 / 5e-2 absolute and relative) and,
being fp32 sums in another order, also at a much tighter one: within one
bf16 rounding step of the oracle's float sum (bf16 out) or 1e-5 relative
(fp32 out).  Larger shapes cover every kernel variant (16-byte, pair and
element loads; 1, 2, 4 and 8 rows per workgroup; the MFMA GEMM with ragged
token and output tiles) and check that nothing past num_tokens * M is
written.  At full projection sizes the check is a torch fp32 product.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu

SENTINEL = 0x7F11


def order_slack(w_f32, x_f32):
    """Room for fp32 sums taken in another order: 2^-20 * sum_n |w||x| per
    output (16 float epsilons of the absolute sum), [tokens][M] flattened."""
    return oracle.gemv(np.abs(w_f32), np.abs(x_f32), nthreads=8).reshape(-1) * 2.0 ** -20


def tight_bf16(got_bits, exp_f32, slack, label):
    """|got - exp| <= one bf16 rounding step of exp (2^-8 relative) + slack."""
    got = H.bf16_bits_to_f32(got_bits).astype(np.float64).reshape(-1)
    exp = exp_f32.astype(np.float64).reshape(-1)
    bad = np.abs(got - exp) > np.abs(exp) * 2.0 ** -8 + slack
    assert not bad.any(), (f"{label}: {int(bad.sum())} outputs off by more than one bf16 step, "
                           f"first {np.flatnonzero(bad)[:4]}")


def tight_f32(got, exp_f32, slack, label):
    got = np.asarray(got, np.float64).reshape(-1)
    exp = exp_f32.astype(np.float64).reshape(-1)
    bad = np.abs(got - exp) > np.abs(exp) * 1e-6 + slack
    assert not bad.any(), f"{label}: {int(bad.sum())} outputs off, first {np.flatnonzero(bad)[:4]}"


def run_bf16(dev, w_bits, x_bits, M, N, tokens, buf, batch_entry):
    wd, xd = H.to_dev_bf16(w_bits, dev), H.to_dev_bf16(x_bits, dev)
    y = torch.full((buf,), SENTINEL, dtype=torch.int16, device=dev)
    if batch_entry:
        attn.batch_gemv_proj_bf16(wd, xd, y, tokens, M, N)
    else:
        attn.gemv_proj_bf16(wd, xd, y, M, N)
    H.sync()
    return y.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("M,N,buf,xp,wp", [(1, 2, 4, 0.17, 0.01), (9, 256, 12, 0.07, 0.006),
                                           (513, 514, 520, 0.05, 0.004)])
def test_gemv_proj_bf16_reference_cases(dev, M, N, buf, xp, wp):
    print(f"[step] gemv bf16 ref case {M}x{N}", flush=True)
    x, w = oracle.make_gemv_case(M, N, xp, wp)
    xb, wb = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
    exp = oracle.gemv(oracle.bf16_to_f32(wb), oracle.bf16_to_f32(xb))
    got = run_bf16(dev, wb, xb, M, N, 1, buf, False)
    H.check_close(H.bf16_bits_to_f32(got[:M]), oracle.round_bf16(exp), 8e-2, 8e-2, "y")
    tight_bf16(got[:M], exp, order_slack(oracle.bf16_to_f32(wb), oracle.bf16_to_f32(xb)), "y")
    assert (got[M:] == SENTINEL).all(), "wrote past M"


@pytest.mark.parametrize("M,N,buf,xp,wp", [(3, 2, 5, 0.19, 0.02), (17, 514, 21, 0.09, 0.005),
                                           (257, 1024, 260, 0.04, 0.003)])
def test_gemv_proj_bf162float_reference_cases(dev, M, N, buf, xp, wp):
    print(f"[step] gemv f32 ref case {M}x{N}", flush=True)
    x, w = oracle.make_gemv_case(M, N, xp, wp)
    xb, wb = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
    exp = oracle.gemv(oracle.bf16_to_f32(wb), oracle.bf16_to_f32(xb))
    y = torch.full((buf,), 1234.5, dtype=torch.float32, device=dev)
    attn.gemv_proj_bf162float(H.to_dev_bf16(wb, dev), H.to_dev_bf16(xb, dev), y, M, N)
    H.sync()
    got = y.cpu().numpy()
    H.check_close(got[:M], exp, 5e-2, 5e-2, "y")
    tight_f32(got[:M], exp, order_slack(oracle.bf16_to_f32(wb), oracle.bf16_to_f32(xb)), "y")
    assert (got[M:] == 1234.5).all(), "wrote past M"


@pytest.mark.parametrize("batch,M,N,hp,wp", [(2, 3, 4, 0.19, 0.12), (4, 12, 20, 0.08, 0.06)])
def test_batch_gemv_proj_reference_cases(dev, batch, M, N, hp, wp):
    print(f"[step] batch gemv ref case {batch}x{M}x{N}", flush=True)
    h, w = oracle.make_batch_gemv_case(batch, M, N, hp, wp)
    hb, wb = oracle.f32_to_bf16(h), oracle.f32_to_bf16(w)
    exp = oracle.gemv(oracle.bf16_to_f32(wb), oracle.bf16_to_f32(hb)).reshape(-1)
    got = run_bf16(dev, wb, hb, M, N, batch, batch * M + 3, True)
    H.check_close(H.bf16_bits_to_f32(got[:batch * M]), oracle.round_bf16(exp), 8e-2, 8e-2, "y")
    tight_bf16(got[:batch * M], exp, order_slack(oracle.bf16_to_f32(wb), oracle.bf16_to_f32(hb)),
               "y")
    assert (got[batch * M:] == SENTINEL).all()


def seeded(seed, M, N, tokens):
    w = synth.uniform_bf16(seed, "w", (M, N), -0.1, 0.1)
    x = synth.normal_bf16(seed, "x", (tokens, N))
    return w, x


# (M, N): 8/4/2/1 rows per workgroup on 16-byte loads, then pair loads
# (N % 8 != 0) and element loads (odd N).
@pytest.mark.parametrize("M,N", [(4096, 4096), (2048, 1024), (1024, 4096), (100, 2048),
                                 (4099, 520), (300, 514), (37, 513)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_gemv_shapes(dev, M, N, out):
    print(f"[step] gemv {out} {M}x{N}", flush=True)
    w, x = seeded(31, M, N, 1)
    wf, xf = H.bf16_bits_to_f32(w), H.bf16_bits_to_f32(x[0])
    exp = oracle.gemv(wf, xf, nthreads=8)
    slack = order_slack(wf, xf)
    wd, xd = H.to_dev_bf16(w, dev), H.to_dev_bf16(x[0], dev)
    if out == "bf16":
        y = torch.full((M + 5,), SENTINEL, dtype=torch.int16, device=dev)
        attn.gemv_proj_bf16(wd, xd, y, M, N)
        H.sync()
        got = y.cpu().numpy().view(np.uint16)
        tight_bf16(got[:M], exp, slack, "y")
        assert (got[M:] == SENTINEL).all()
    else:
        y = torch.full((M + 5,), 1234.5, dtype=torch.float32, device=dev)
        attn.gemv_proj_bf162float(wd, xd, y, M, N)
        H.sync()
        got = y.cpu().numpy()
        tight_f32(got[:M], exp, slack, "y")
        assert (got[M:] == 1234.5).all()


def test_gemv_unaligned_operands(dev):
    """W and x at 2-byte offsets (element loads) and at 4-byte offsets (pair
    loads) give the same result as aligned operands."""
    M, N = 257, 1024
    w, x = seeded(32, M, N, 1)
    wf, xf = H.bf16_bits_to_f32(w), H.bf16_bits_to_f32(x[0])
    exp, slack = oracle.gemv(wf, xf), order_slack(wf, xf)
    for off in (1, 2):
        wbuf = torch.zeros(M * N + off, dtype=torch.int16, device=dev)
        xbuf = torch.zeros(N + off, dtype=torch.int16, device=dev)
        wbuf[off:] = H.to_dev_bf16(w, dev).view(torch.int16).reshape(-1)
        xbuf[off:] = H.to_dev_bf16(x[0], dev).view(torch.int16)
        y = torch.full((M,), SENTINEL, dtype=torch.int16, device=dev)
        attn.gemv_proj_bf16(wbuf[off:], xbuf[off:], y, M, N)
        H.sync()
        tight_bf16(y.cpu().numpy().view(np.uint16), exp, slack, f"offset {off}")


# Token counts on both sides of the GEMV/GEMM switch (T > 4 with N % 64 == 0),
# ragged token and output tiles, and N % 64 != 0 (GEMV over token groups).
@pytest.mark.parametrize("T,M,N", [(1, 512, 1024), (3, 1000, 1024), (4, 256, 2048),
                                   (5, 384, 1024), (17, 200, 1024), (128, 256, 512),
                                   (300, 1000, 1024), (129, 130, 64), (40, 96, 520),
                                   (9, 77, 514)])
def test_batch_proj_shapes(dev, T, M, N):
    print(f"[step] batch proj T={T} M={M} N={N}", flush=True)
    w, x = seeded(33, M, N, T)
    wf, xf = H.bf16_bits_to_f32(w), H.bf16_bits_to_f32(x)
    exp = oracle.gemv(wf, xf, nthreads=8).reshape(-1)
    got = run_bf16(dev, w, x, M, N, T, T * M + 7, True)
    tight_bf16(got[:T * M], exp, order_slack(wf, xf), "y")
    assert (got[T * M:] == SENTINEL).all()


# The first two tile the chip with 256 x 256 tiles, with ragged tiles and
# slice counts that are odd or tiny; 1371 x 6144 takes the 128 x 192 tiles
# (its 128 x 128 grid would overflow the resident workgroups).
@pytest.mark.parametrize("T,M,N", [(4096, 4096, 4096), (4000, 4100, 4160), (4096, 4096, 64),
                                   (2048, 4096, 4096), (1000, 1024, 4096), (512, 12288, 4096),
                                   (512, 4096, 12288), (1371, 6144, 1024)])
def test_batch_proj_full_size_vs_torch_fp32(dev, T, M, N):
    """Prefill projection shapes of an 8B model against a torch fp32 product
    of the same bf16 inputs."""
    print(f"[step] batch proj full T={T} M={M} N={N}", flush=True)
    g = torch.Generator(device=dev).manual_seed(34)
    w = (torch.randn((M, N), generator=g, device=dev) * 0.03).to(torch.bfloat16)
    x = torch.randn((T, N), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((T, M), dtype=torch.bfloat16, device=dev)
    attn.batch_gemv_proj_bf16(w, x, y, T, M, N)
    ref = x.float() @ w.float().t()
    slack = (x.float().abs() @ w.float().abs().t()) * 2.0 ** -20
    H.sync()
    err = (y.float() - ref).abs()
    assert bool((err <= ref.abs() * 2.0 ** -8 + slack).all()), f"max err {float(err.max())}"


def test_batch_proj_graph_replay(dev):
    """Captured once, replayed with new inputs: each replay matches the eager call."""
    T, M, N = 256, 512, 1024
    w, x = seeded(35, M, N, T)
    wd, xd = H.to_dev_bf16(w, dev), H.to_dev_bf16(x, dev)
    y = torch.empty((T, M), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        attn.batch_gemv_proj_bf16(wd, xd, y, T, M, N, stream)
    H.sync()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        attn.batch_gemv_proj_bf16(wd, xd, y, T, M, N, stream)
    for k in range(3):
        xd.copy_(H.to_dev_bf16(synth.normal_bf16(36 + k, "x", (T, N)), dev))
        y.zero_()
        H.sync()
        graph.replay()
        H.sync()
        ref = torch.empty_like(y)
        attn.batch_gemv_proj_bf16(wd, xd, ref, T, M, N)
        H.sync()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"replay {k}"


@pytest.mark.parametrize("T,hid,rows", [(1371, 1024, (2048, 1024, 1024)), (4096, 1024, (2048, 1024, 1024)),
                                      (300, 512, (3072, 3072)), (1371, 1024, (3072, 3072)),
                                      (17, 256, (200, 64, 130))])
def test_gemm_segments_equal_separate_projections(dev, T, hid, rows):
    """Stacked segments in one launch (whichever tile size the stacked grid
    picks) give each element bit for bit what the separate projection gives:
    every tile size sums k in the same MFMA order."""
    print(f"[step] gemm segments T={T} hid={hid} rows={rows}", flush=True)
    g = torch.Generator(device=dev).manual_seed(37)
    x = torch.randn((T, hid), generator=g, device=dev).to(torch.bfloat16)
    ws = [(torch.randn((r, hid), generator=g, device=dev) * 0.05).to(torch.bfloat16) for r in rows]
    ys = [torch.empty((T, r), dtype=torch.bfloat16, device=dev) for r in rows]
    attn.gemm_segments_bf16(x, T, hid, ws, ys, rows)
    for w, y, r in zip(ws, ys, rows):
        ref = torch.empty_like(y)
        attn.batch_gemv_proj_bf16(w, x, ref, T, r, hid)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"rows {r}"


@pytest.mark.parametrize("T,H,M", [(700, 2048, 1024), (129, 512, 130)])
def test_gemm_residual_epilogue_equals_projection_then_add(dev, T, H, M):
    """residual != 0: y = bf16(y + bf16(x W^T)), bit for bit the projection
    followed by residual_add_bf16 (M = 130: rows not 16-byte aligned, so the
    epilogue's element stores)."""
    print(f"[step] gemm residual T={T} H={H} M={M}", flush=True)
    g = torch.Generator(device=dev).manual_seed(38)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((M, H), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    hid = torch.randn((T, M), generator=g, device=dev).to(torch.bfloat16)
    fused = hid.clone()
    attn.gemm_segments_bf16(x, T, H, [w], [fused], [M], residual=True)
    proj = torch.empty((T, M), dtype=torch.bfloat16, device=dev)
    attn.batch_gemv_proj_bf16(w, x, proj, T, M, H)
    ref = hid.clone()
    attn.batch_residual_add_bf16(proj, ref, T, M)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))



@pytest.mark.parametrize("T,hid,M", [(1371, 1024, 3072), (4096, 1024, 3072), (300, 512, 3072),
                                     (17, 256, 200), (33, 256, 204)])
def test_gemm_swiglu_equals_projections_then_swiglu(dev, T, hid, M):
    """Gate/up with SwiGLU in the GEMM epilogue (192 x 128, 256 x 256 and
    128 x 128 tiles by grid size; a ragged last tile at M = 200; M = 204:
    rows not 16-byte aligned) equals the two projections followed by
    batch_swiglu_bf16x2, bit for bit."""
    print(f"[step] gemm swiglu T={T} hid={hid} M={M}", flush=True)
    g = torch.Generator(device=dev).manual_seed(39)
    x = torch.randn((T, hid), generator=g, device=dev).to(torch.bfloat16)
    wg = (torch.randn((M, hid), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    wu = (torch.randn((M, hid), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    out = torch.full((T, M), -7.0, dtype=torch.bfloat16, device=dev)
    attn.gemm_swiglu_bf16(x, T, hid, wg, wu, M, out)
    gate = torch.empty((T, M), dtype=torch.bfloat16, device=dev)
    up = torch.empty_like(gate)
    attn.batch_gemv_proj_bf16(wg, x, gate, T, M, hid)
    attn.batch_gemv_proj_bf16(wu, x, up, T, M, hid)
    ref = torch.empty_like(gate)
    attn.batch_swiglu_bf16x2(gate, up, ref, T, M)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
