"""The rest of a Qwen3 decoder layer vs the oracle: full-row RMSNorm (single
and batched, with the `sum` output), residual add, SwiGLU, embedding gather and
argmax, through the C ABI.

Bars: the reference tests' 2e-2 absolute and relative
(tests/test_rmsnorm_bf16.cu:40-46 with the sum at 5e-2 / 5e-3,
tests/test_swiglu_bf16x2.cu:36, tests/test_residual_add_bf16.cu:26-42 and the
batch tests), and, because both sides round the same fp32 value once,
within one bf16 rounding step of the oracle (RMSNorm's device rsqrt and
fmaf(sum, 1/size, eps) differ from the host's 1/sqrt(sum/size + eps) in the
last float bits; exp likewise).  Residual add, gather and argmax are exact.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu

SENTINEL = 0x7F11


def bf16(x):
    return oracle.f32_to_bf16(np.asarray(x, np.float32))


def within_step(got_bits, exp_f32, label):
    got = H.bf16_bits_to_f32(got_bits).astype(np.float64)
    exp = np.asarray(exp_f32, np.float64)
    bad = np.abs(got - exp) > np.abs(exp) * 2.0 ** -7 + 1e-30
    assert not bad.any(), f"{label}: {int(bad.sum())} off by more than one bf16 step"


def run_rmsnorm(dev, xb, wb, rows, size, eps, out_len, batch):
    x, w = H.to_dev_bf16(xb, dev), H.to_dev_bf16(wb, dev)
    y = torch.full((out_len,), SENTINEL, dtype=torch.int16, device=dev)
    s = torch.full((rows + 1,), -123.0, dtype=torch.float32, device=dev)
    if batch:
        attn.batch_rmsnorm_bf16(x, w, y, s, eps, rows, size)
    else:
        attn.rmsnorm_bf16(x, w, y, s, eps, size)
    H.sync()
    return y.cpu().numpy().view(np.uint16), s.cpu().numpy()


def rmsnorm_cases():
    tiny_x = [0.0, -1.25, 0.75, -0.5, 1.0, -1.5]
    tiny_w = [1.0, -0.75, 0.25, -1.25, 0.5, 0.875]
    yield "tiny", 2, 6, 1e-5, np.array(tiny_x, np.float32), np.array(tiny_w, np.float32)
    for label, size, buf, eps, ip, wp in (("partial-block", 258, 264, 1e-5, 0.11, 0.07),
                                          ("multi-block", 1024, 1030, 1e-3, 0.07, 0.03)):
        x, w = oracle.make_rmsnorm_row_case(size, buf, ip, wp)
        yield label, size, buf, eps, x, w
    w = np.array([-1.2 + 0.01 * ((i * 9) % 23) for i in range(520)], np.float32)
    yield "zero-input", 514, 520, 1e-4, np.zeros(520, np.float32), w


@pytest.mark.parametrize("case", list(rmsnorm_cases()), ids=lambda c: c[0])
def test_rmsnorm_reference_cases(dev, case):
    """tests/test_rmsnorm_bf16.cu:60-90: output past `size` untouched, sum =
    the sum of squares (initialised to -123 first)."""
    label, size, buf, eps, x, w = case
    xb, wb = bf16(x), bf16(w)
    exp = oracle.rmsnorm_rows(H.bf16_bits_to_f32(xb[:size]), H.bf16_bits_to_f32(wb[:size]), eps)
    got, s = run_rmsnorm(dev, xb, wb, 1, size, eps, buf, False)
    H.check_close(H.bf16_bits_to_f32(got[:size]), exp, 2e-2, 2e-2, label)
    within_step(got[:size], exp, label)
    assert (got[size:] == SENTINEL).all()
    ref_sum = float(np.sum(H.bf16_bits_to_f32(xb[:size]).astype(np.float64) ** 2))
    assert abs(s[0] - ref_sum) <= 5e-2 + 5e-3 * abs(ref_sum), (s[0], ref_sum)


@pytest.mark.parametrize("batch,size,eps,ip,wp", [(1, 16, 1e-5, 0.15, 0.22),
                                                  (3, 32, 1e-4, 0.08, 0.12)])
def test_batch_rmsnorm_reference_cases(dev, batch, size, eps, ip, wp):
    """tests/test_batch_rmsnorm_bf16.cu:100-106."""
    x, w = oracle.make_batch_row_rmsnorm_case(batch, size, ip, wp)
    xb, wb = bf16(x), bf16(w)
    exp = oracle.rmsnorm_rows(H.bf16_bits_to_f32(xb), H.bf16_bits_to_f32(wb), eps)
    got, s = run_rmsnorm(dev, xb.reshape(-1), wb, batch, size, eps, batch * size + 4, True)
    H.check_close(H.bf16_bits_to_f32(got[:batch * size]), exp.reshape(-1), 2e-2, 2e-2, "y")
    within_step(got[:batch * size], exp.reshape(-1), "y")
    assert (got[batch * size:] == SENTINEL).all()
    sums = (H.bf16_bits_to_f32(xb).astype(np.float64) ** 2).sum(axis=1)
    assert np.allclose(s[:batch], sums, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rows,size", [(1371, 1024), (4, 4096), (3, 1030), (2, 12288), (5, 6)])
def test_rmsnorm_shapes(dev, rows, size):
    """Prefill and decode widths on the 16-byte path, and the pair path
    (size % 8 != 0); in place as well."""
    xb = synth.normal_bf16(41, "x", (rows, size))
    wb = synth.uniform_bf16(41, "w", (size,), 0.5, 1.5)
    exp = oracle.rmsnorm_rows(H.bf16_bits_to_f32(xb), H.bf16_bits_to_f32(wb), 1e-6)
    got, _ = run_rmsnorm(dev, xb.reshape(-1), wb, rows, size, 1e-6, rows * size, True)
    within_step(got, exp.reshape(-1), "y")
    x = H.to_dev_bf16(xb, dev)
    attn.batch_rmsnorm_bf16(x, H.to_dev_bf16(wb, dev), x, None, 1e-6, rows, size)
    H.sync()
    assert np.array_equal(H.from_dev_bf16(x).reshape(-1), got), "in place differs"


@pytest.mark.parametrize("size,buf,twice,rp,hp,tail", [(6, 6, True, None, None, None),
                                                       (514, 520, False, 0.09, 0.07, 0.6),
                                                       (1536, 1542, True, 0.05, 0.04, -0.45)])
def test_residual_add_reference_cases(dev, size, buf, twice, rp, hp, tail):
    """tests/test_residual_add_bf16.cu:56-66, applied twice where the reference does."""
    if rp is None:
        r = np.array([0.5, -0.25, 1.25, -1.5, 0.75, -0.5], np.float32)
        h = np.array([-1.0, 0.75, -0.125, 0.875, -1.75, 1.5], np.float32)
    else:
        r, h = oracle.make_add_case(size, buf, rp, hp, tail)
    rb, hb = bf16(r), bf16(h)
    rd, hd = H.to_dev_bf16(rb, dev), H.to_dev_bf16(hb, dev)
    exp = H.bf16_bits_to_f32(hb).copy()
    for _ in range(2 if twice else 1):
        attn.residual_add_bf16(rd, hd, size)
        exp[:size] = oracle.residual_add(exp[:size], H.bf16_bits_to_f32(rb[:size]))
    H.sync()
    got = H.from_dev_bf16(hd)
    assert np.array_equal(H.bf16_bits_to_f32(got), exp)


@pytest.mark.parametrize("tokens,size", [(1, 6), (3, 32), (1371, 1024), (7, 1030)])
def test_batch_residual_add(dev, tokens, size):
    rb = synth.normal_bf16(42, "r", (tokens, size))
    hb = synth.normal_bf16(42, "h", (tokens, size))
    hd = H.to_dev_bf16(hb, dev)
    attn.batch_residual_add_bf16(H.to_dev_bf16(rb, dev), hd, tokens, size)
    H.sync()
    exp = oracle.residual_add(H.bf16_bits_to_f32(hb), H.bf16_bits_to_f32(rb))
    assert np.array_equal(H.bf16_bits_to_f32(H.from_dev_bf16(hd)), exp)


def swiglu_cases():
    g = np.array([-2.0, 1.5, 0.25, -1.25, 0.5, -0.75], np.float32)
    u = np.array([0.75, -0.5, 1.0, -1.5, 0.25, -0.125], np.float32)
    yield "tiny", 6, 6, g, u
    for label, size, buf, gp, up in (("partial-block", 514, 520, 0.08, 0.05),
                                     ("multi-block", 2048, 2054, 0.021, 0.017)):
        g, u = oracle.make_swiglu_case(size, buf, gp, up)
        yield label, size, buf, g, u


@pytest.mark.parametrize("case", list(swiglu_cases()), ids=lambda c: c[0])
def test_swiglu_reference_cases(dev, case):
    """tests/test_swiglu_bf16x2.cu:50-60; output past `size` untouched."""
    label, size, buf, g, u = case
    gb, ub = bf16(g), bf16(u)
    exp = oracle.swiglu(H.bf16_bits_to_f32(gb[:size]), H.bf16_bits_to_f32(ub[:size]))
    out = torch.full((buf,), SENTINEL, dtype=torch.int16, device=dev)
    attn.swiglu_bf16x2(H.to_dev_bf16(gb, dev), H.to_dev_bf16(ub, dev), out, size)
    H.sync()
    got = out.cpu().numpy().view(np.uint16)
    H.check_close(H.bf16_bits_to_f32(got[:size]), exp, 2e-2, 2e-2, label)
    within_step(got[:size], exp, label)
    assert (got[size:] == SENTINEL).all()


@pytest.mark.parametrize("tokens,size", [(2, 8), (3, 40), (1371, 3072), (5, 1030)])
def test_batch_swiglu(dev, tokens, size):
    gb = synth.normal_bf16(43, "g", (tokens, size))
    ub = synth.normal_bf16(43, "u", (tokens, size))
    out = torch.empty((tokens, size), dtype=torch.bfloat16, device=dev)
    attn.batch_swiglu_bf16x2(H.to_dev_bf16(gb, dev), H.to_dev_bf16(ub, dev), out, tokens, size)
    H.sync()
    exp = oracle.swiglu(H.bf16_bits_to_f32(gb), H.bf16_bits_to_f32(ub))
    within_step(H.from_dev_bf16(out).reshape(-1), exp.reshape(-1), "y")


@pytest.mark.parametrize("size", [1024, 6, 1030])
def test_gather_embedding(dev, size):
    """Rows copied bit for bit; ids at or past vocab_size give zero rows."""
    vocab = 1000
    table = synth.normal_bf16(44, "e", (vocab, size))
    ids = np.array([0, 999, 17, 17, 500, 1000, 123456], np.uint32)
    out = torch.full((len(ids), size), 1.0, dtype=torch.bfloat16, device=dev)
    ids_d = torch.from_numpy(ids.view(np.int32)).to(dev)
    attn.gather_embedding_bf16(H.to_dev_bf16(table, dev), ids_d, out, len(ids), size, vocab)
    H.sync()
    got = H.from_dev_bf16(out)
    for t, i in enumerate(ids):
        exp = table[i] if i < vocab else np.zeros(size, np.uint16)
        assert np.array_equal(got[t], exp), f"token {t} id {i}"


def test_argmax(dev):
    """First maximum, NaN never wins, ties to the smaller index, nothing above
    -FLT_MAX gives UINT32_MAX; a 151936-entry row as the lm-head produces."""
    rng = np.random.default_rng(9)
    cases = [rng.normal(size=151936).astype(np.float32),
             np.array([1.0, 5.0, 5.0, 2.0], np.float32),
             np.array([np.nan, -1.0, np.nan, 3.0, np.nan], np.float32),
             np.array([-np.inf, np.nan], np.float32)]
    tie = rng.normal(size=5000).astype(np.float32)
    tie[[4000, 1234, 4999]] = 50.0
    cases.append(tie)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    for c in cases:
        attn.argmax_f32(torch.from_numpy(c).to(dev), len(c), out)
        H.sync()
        assert int(out.cpu().numpy().view(np.uint32)[0]) == oracle.argmax(c)
    assert oracle.argmax(tie) == 1234
