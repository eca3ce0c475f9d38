"""GPU parity of the sequence-LIF kernels against the CPU oracle.

Bars (written per test):
* spikes: bit-exact against the reference loop evaluated in float32 on the
  same (widened) inputs -- the kernel does the loop's float32 operations in
  the same order, so membranes and spikes agree exactly;
* dL/dx, fp32 I/O: ``rtol=1e-5`` with ``atol=1e-5 * max|ref|`` against the
  float64 reverse recurrence over the float32 forward's spike pattern;
* dL/dx, bf16/fp16 I/O: ``rtol=2e-2, atol=1e-2 * max|ref|``.
"""

from __future__ import annotations

import pytest
import torch

from oracle import lif as L

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: (1e-5, 1e-5), torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-2, 1e-2)}


def _ops():
    import spikegpt_myelin_amd  # noqa: F401

    return torch.ops.myelin


def _inputs(b, t, c, dtype, seed=0, scale=1.5):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(b, t, c, generator=g) * scale).to(dtype)
    gs = torch.randn(b, t, c, generator=g).to(dtype)
    return x, gs


def _check_grad(got, ref, dtype, what):
    rtol, atol_scale = TOL[dtype]
    got = got.double().cpu()
    ref = ref.double()
    atol = atol_scale * max(float(ref.abs().max()) if ref.numel() else 0.0, 1.0)
    err = float((got - ref).abs().max()) if ref.numel() else 0.0
    assert torch.allclose(got, ref, rtol=rtol, atol=atol), f"{what}: max abs err {err:.3e}"


def _run(x, gs, tau=2.0, threshold=1.0, reset=0.0, slope=2.0):
    ops = _ops()
    decay = 1.0 - 1.0 / tau
    xd = x.to(DEV)
    spikes, ck = ops.lif_sequence_forward(xd, decay, threshold, reset, slope)
    gx = ops.lif_sequence_backward(gs.to(DEV), xd, ck, decay, threshold, reset, slope)
    torch.cuda.synchronize()
    return spikes.cpu(), gx.cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(3, 1, 96), (3, 7, 96), (2, 64, 128), (2, 100, 70),
                                   (1, 33, 129), (4, 257, 256)])
def test_forward_and_backward_match_oracle(dtype, shape):
    b, t, c = shape
    x, gs = _inputs(b, t, c, dtype, seed=b * 1000 + t + c)
    spikes, gx = _run(x, gs)
    ref_s = L.lif_loop(x.float()).to(dtype)
    assert spikes.dtype == dtype
    assert torch.equal(spikes, ref_s), f"spikes differ at {shape} {dtype}"
    ref_g = L.lif_reverse(x.float(), gs.float(), forward_dtype=torch.float32)
    _check_grad(gx, ref_g, dtype, f"grad_x {shape} {dtype}")


@pytest.mark.parametrize("params", [dict(tau=3.0, threshold=0.7, reset=-0.25, slope=1.5),
                                    dict(tau=1.25, threshold=1.2, reset=0.1, slope=4.0)])
def test_neuron_parameters(params):
    x, gs = _inputs(2, 130, 192, torch.float32, seed=7)
    spikes, gx = _run(x, gs, **params)
    assert torch.equal(spikes, L.lif_loop(x, params["tau"], params["threshold"], params["reset"],
                                          params["slope"]))
    ref_g = L.lif_reverse(x, gs, params["tau"], params["threshold"], params["reset"],
                          params["slope"], forward_dtype=torch.float32)
    _check_grad(gx, ref_g, torch.float32, f"grad_x {params}")


def test_autograd_through_the_op_and_module():
    from spikegpt_myelin_amd import lif_sequence
    from spikegpt_myelin_amd.model import SpikingSequenceLIF

    x, gs = _inputs(2, 90, 160, torch.bfloat16, seed=11)
    xd = x.to(DEV).requires_grad_(True)
    s = SpikingSequenceLIF(tau=2.0)(xd)
    (gx,) = torch.autograd.grad(s, xd, gs.to(DEV))
    assert torch.equal(s.detach().cpu(), L.lif_loop(x.float()).to(torch.bfloat16))
    _check_grad(gx, L.lif_reverse(x.float(), gs.float(), forward_dtype=torch.float32),
                torch.bfloat16, "module grad")
    # The functional form gives the same bits.
    s2 = lif_sequence(xd.detach())
    assert torch.equal(s2, s.detach())


def test_empty_inputs():
    ops = _ops()
    for shape in [(0, 5, 8), (2, 0, 8), (2, 5, 0)]:
        x = torch.zeros(shape, device=DEV)
        s, ck = ops.lif_sequence_forward(x, 0.5, 1.0, 0.0, 2.0)
        assert s.shape == x.shape
        gx = ops.lif_sequence_backward(torch.zeros_like(x), x, ck, 0.5, 1.0, 0.0, 2.0)
        assert gx.shape == x.shape


def test_bad_parameters_raise():
    ops = _ops()
    x = torch.zeros(1, 4, 8, device=DEV)
    with pytest.raises(RuntimeError, match="surrogate_slope positive"):
        ops.lif_sequence_forward(x, 0.5, 1.0, 0.0, 0.0)
    with pytest.raises(ValueError, match=r"\[B, T, C\]"):
        ops.lif_sequence_forward(torch.zeros(4, 8, device=DEV), 0.5, 1.0, 0.0, 2.0)


def test_benchmark_shape_full_size():
    # B=64, T=1024, C=512 bf16 (the 41M model's activation shape; two
    # channels per lane): exact spikes and gradients against the oracle.
    x, gs = _inputs(64, 1024, 512, torch.bfloat16, seed=3, scale=1.0)
    spikes, gx = _run(x, gs)
    assert torch.equal(spikes, L.lif_loop(x.float()).to(torch.bfloat16))
    rate = float(spikes.float().mean())
    assert 0.01 < rate < 0.9
    _check_grad(gx, L.lif_reverse(x.float(), gs.float(), forward_dtype=torch.float32),
                torch.bfloat16, "grad_x full size")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 100, 64), (3, 257, 256), (1, 5, 8)])
def test_residual_forward_and_backward(dtype, shape):
    # out = residual + spikes(x) (exact), d out/d residual = identity,
    # d out/d x = the LIF backward of an fp32 gradient.
    from spikegpt_myelin_amd.lif import lif_residual

    b, t, c = shape
    x, _ = _inputs(b, t, c, dtype, seed=b + t + c)
    g = torch.Generator().manual_seed(5)
    residual = torch.randn(b, t, c, generator=g)
    gout = torch.randn(b, t, c, generator=g)
    xd = x.to(DEV).requires_grad_(True)
    rd = residual.to(DEV).requires_grad_(True)
    out = lif_residual(rd, xd)
    assert out.dtype == torch.float32
    spikes = L.lif_loop(x.float())
    assert torch.equal(out.detach().cpu(), residual + spikes), f"out differs at {shape} {dtype}"
    gx, gr = torch.autograd.grad(out, (xd, rd), gout.to(DEV))
    assert torch.equal(gr.cpu(), gout)
    ref = L.lif_reverse(x.float(), gout, forward_dtype=torch.float32)
    _check_grad(gx, ref, dtype, f"residual grad_x {shape} {dtype}")


def test_residual_full_size():
    from spikegpt_myelin_amd.lif import lif_residual

    x, _ = _inputs(64, 1024, 512, torch.bfloat16, seed=9, scale=1.0)
    g = torch.Generator().manual_seed(6)
    residual = torch.randn(64, 1024, 512, generator=g)
    gout = torch.randn(64, 1024, 512, generator=g)
    xd = x.to(DEV).requires_grad_(True)
    out = lif_residual(residual.to(DEV), xd)
    assert torch.equal(out.detach().cpu(), residual + L.lif_loop(x.float()))
    (gx,) = torch.autograd.grad(out, xd, gout.to(DEV))
    _check_grad(gx, L.lif_reverse(x.float(), gout, forward_dtype=torch.float32),
                torch.bfloat16, "residual grad_x full size")


# Split over time of the forward: segments run at once from a guessed
# membrane and a repair pass makes them exact, so every output and record
# must equal the one-pass kernel's bit for bit.  Parameter sets: the model's
# (the runs converge within the warm-up), a negative decay (tau 0.7), and a
# slow leak with a constant drive (tau 100: the guessed and exact runs spike
# with different phases and never coincide, so the repair reruns whole
# segments).
LIF_PARAMS = {
    "model": dict(tau=2.0, threshold=1.0, reset=0.0, slope=2.0, scale=1.5, const=None),
    "negative_decay": dict(tau=0.7, threshold=1.0, reset=-0.5, slope=2.0, scale=1.5, const=None),
    "no_convergence": dict(tau=100.0, threshold=1.0, reset=0.0, slope=2.0, scale=0.0,
                           const=0.02),
}


def _lif_case(b, t, c, dtype, kind, seed):
    p = LIF_PARAMS[kind]
    if p["const"] is not None:
        x = torch.full((b, t, c), p["const"]).to(dtype)
        # channels start from different drives so their phases differ
        x = (x.float() * (1 + torch.arange(c) / (2 * c))).to(dtype)
    else:
        x, _ = _inputs(b, t, c, dtype, seed=seed, scale=p["scale"])
    return x, p


def _forward(x, p):
    ops = _ops()
    s, ck = ops.lif_sequence_forward(x.to(DEV), 1.0 - 1.0 / p["tau"], p["threshold"], p["reset"],
                                     p["slope"])
    torch.cuda.synchronize()
    return s.cpu(), ck.cpu()


@pytest.mark.parametrize("kind", list(LIF_PARAMS))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 100, 70), (3, 257, 256), (1, 1000, 128), (2, 300, 136)])
def test_split_forward_equals_one_pass(kind, dtype, shape, monkeypatch):
    b, t, c = shape
    x, p = _lif_case(b, t, c, dtype, kind, seed=t + c)
    print(f"lif split {kind} {dtype} {shape}", flush=True)
    monkeypatch.setenv("WKV_LIF_SEGS", "1")
    s1, ck1 = _forward(x, p)
    ref = L.lif_loop(x.float(), p["tau"], p["threshold"], p["reset"], p["slope"]).to(dtype)
    assert torch.equal(s1, ref)
    for segs in ("2", "3", "5", "16"):
        for warm in ("0", "1", "2"):
            monkeypatch.setenv("WKV_LIF_SEGS", segs)
            monkeypatch.setenv("WKV_LIF_WARMUP", warm)
            s2, ck2 = _forward(x, p)
            assert torch.equal(s2, s1), f"spikes: {segs} segments, warm-up {warm}"
            assert torch.equal(ck2.view(torch.int32), ck1.view(torch.int32)), \
                f"records: {segs} segments, warm-up {warm}"


@pytest.mark.parametrize("kind", list(LIF_PARAMS))
@pytest.mark.parametrize("shape", [(2, 100, 64), (3, 257, 256), (1, 1000, 136)])
def test_split_residual_forward_equals_one_pass(kind, shape, monkeypatch):
    from spikegpt_myelin_amd import _lib

    ops = _ops()
    b, t, c = shape
    x, p = _lif_case(b, t, c, torch.bfloat16, kind, seed=b + t)
    residual = torch.randn(b, t, c, generator=torch.Generator().manual_seed(t))
    decay = 1.0 - 1.0 / p["tau"]
    args = (decay, p["threshold"], p["reset"], p["slope"])
    print(f"lif residual split {kind} {shape}", flush=True)
    monkeypatch.setenv("WKV_LIF_SEGS", "1")
    o1, ck1 = ops.lif_residual_forward(x.to(DEV), residual.to(DEV), *args)
    spikes = L.lif_loop(x.float(), p["tau"], p["threshold"], p["reset"], p["slope"])
    assert torch.equal(o1.cpu(), residual + spikes)
    for segs in ("2", "5", "16"):
        monkeypatch.setenv("WKV_LIF_SEGS", segs)
        o2, ck2 = ops.lif_residual_forward(x.to(DEV), residual.to(DEV), *args)
        assert torch.equal(o2, o1), f"out: {segs} segments"
        assert torch.equal(ck2.view(torch.int32), ck1.view(torch.int32)), f"records: {segs}"
    # In place (out aliasing the residual) through the C ABI: the one-pass
    # kernel runs whatever the workspace, with the same result.
    lib = _lib.load()
    inplace = residual.to(DEV).clone()
    xd = x.to(DEV)
    ck = torch.empty_like(ck1, device=DEV)
    nbytes = int(lib.lif_forward_workspace_bytes(b, t, c))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    _lib.check(lib.lif_residual_forward(
        xd.data_ptr(), inplace.data_ptr(), inplace.data_ptr(), ck.data_ptr(), ws.data_ptr(), nbytes,
        b, t, c, *args, _lib.dtype_code(xd.dtype), torch.cuda.current_stream().cuda_stream),
        "lif_residual_forward in place")
    torch.cuda.synchronize()
    assert torch.equal(inplace, o1)
    assert torch.equal(ck.cpu().view(torch.int32), ck1.cpu().view(torch.int32))


def test_default_split_at_the_benchmark_shape():
    # B=64, T=1024, C=512: the sizes alone pick the split (eight segments),
    # and the full-size tests above ran it.
    from spikegpt_myelin_amd import _lib

    assert int(_lib.load().lif_forward_workspace_bytes(64, 1024, 512)) == 2 * 7 * 64 * 512 * 4


@pytest.mark.parametrize("kind", list(LIF_PARAMS))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 100, 70), (3, 257, 256), (1, 1000, 128), (2, 300, 136)])
def test_split_backward_equals_one_pass(kind, dtype, shape, monkeypatch):
    # The backward's split mirrors the forward's (segments run last to
    # first from a zero gradient carry after a warm-up, then a repair pass):
    # dL/dx bit-identical to the one-pass kernel, and to the oracle's bar.
    ops = _ops()
    b, t, c = shape
    x, p = _lif_case(b, t, c, dtype, kind, seed=t + c + 1)
    gs = torch.randn(b, t, c, generator=torch.Generator().manual_seed(c)).to(dtype)
    decay = 1.0 - 1.0 / p["tau"]
    args = (decay, p["threshold"], p["reset"], p["slope"])
    print(f"lif backward split {kind} {dtype} {shape}", flush=True)
    monkeypatch.setenv("WKV_LIF_SEGS", "1")
    _, ck = ops.lif_sequence_forward(x.to(DEV), *args)
    monkeypatch.setenv("WKV_LIF_BWD_SEGS", "1")
    g1 = ops.lif_sequence_backward(gs.to(DEV), x.to(DEV), ck, *args).cpu()
    ref = L.lif_reverse(x.float(), gs.float(), p["tau"], p["threshold"], p["reset"], p["slope"],
                        forward_dtype=torch.float32)
    _check_grad(g1, ref, dtype, f"one pass {kind}")
    for segs in ("2", "3", "5", "16"):
        for warm in ("0", "1", "2"):
            monkeypatch.setenv("WKV_LIF_BWD_SEGS", segs)
            monkeypatch.setenv("WKV_LIF_BWD_WARMUP", warm)
            g2 = ops.lif_sequence_backward(gs.to(DEV), x.to(DEV), ck, *args).cpu()
            assert torch.equal(g2.view(torch.int16 if dtype != torch.float32 else torch.int32),
                               g1.view(torch.int16 if dtype != torch.float32 else torch.int32)), \
                f"grad_x: {segs} segments, warm-up {warm}"


@pytest.mark.parametrize("kind", list(LIF_PARAMS))
def test_split_residual_backward_equals_one_pass(kind, monkeypatch):
    ops = _ops()
    b, t, c = 2, 1000, 136
    x, p = _lif_case(b, t, c, torch.bfloat16, kind, seed=7)
    g = torch.randn(b, t, c, generator=torch.Generator().manual_seed(8))
    residual = torch.zeros(b, t, c)
    args = (1.0 - 1.0 / p["tau"], p["threshold"], p["reset"], p["slope"])
    print(f"lif residual backward split {kind}", flush=True)
    _, ck = ops.lif_residual_forward(x.to(DEV), residual.to(DEV), *args)
    monkeypatch.setenv("WKV_LIF_BWD_SEGS", "1")
    g1 = ops.lif_residual_backward(g.to(DEV), x.to(DEV), ck, *args).cpu()
    for segs in ("2", "5", "16"):
        monkeypatch.setenv("WKV_LIF_BWD_SEGS", segs)
        g2 = ops.lif_residual_backward(g.to(DEV), x.to(DEV), ck, *args).cpu()
        assert torch.equal(g2.view(torch.int16), g1.view(torch.int16)), f"{segs} segments"


def test_default_backward_split_at_the_benchmark_shape():
    from spikegpt_myelin_amd import _lib

    # four segments of eight blocks
    assert int(_lib.load().lif_backward_workspace_bytes(64, 1024, 512)) == 2 * 3 * 64 * 512 * 4


def test_216m_activation_shape_with_the_default_split():
    # B=16, T=1024, C=768 bf16 (the 216M class): the sizes alone pick the
    # split (forward 8 segments, backward 4; the residual forward also 8 at
    # these 192 rows).  Spikes exact, gradients to the 16-bit bar, and the
    # residual form equal to residual + spikes.
    from spikegpt_myelin_amd import _lib
    from spikegpt_myelin_amd.lif import lif_residual

    b, t, c = 16, 1024, 768
    lib = _lib.load()
    assert int(lib.lif_forward_workspace_bytes(b, t, c)) == 2 * 7 * b * c * 4
    assert int(lib.lif_backward_workspace_bytes(b, t, c)) == 2 * 3 * b * c * 4
    x, gs = _inputs(b, t, c, torch.bfloat16, seed=21, scale=1.0)
    spikes, gx = _run(x, gs)
    assert torch.equal(spikes, L.lif_loop(x.float()).to(torch.bfloat16))
    _check_grad(gx, L.lif_reverse(x.float(), gs.float(), forward_dtype=torch.float32),
                torch.bfloat16, "grad_x 216M shape")
    residual = torch.randn(b, t, c, generator=torch.Generator().manual_seed(22))
    gout = torch.randn(b, t, c, generator=torch.Generator().manual_seed(23))
    xd = x.to(DEV).requires_grad_(True)
    out = lif_residual(residual.to(DEV), xd)
    assert torch.equal(out.detach().cpu(), residual + L.lif_loop(x.float()))
    (gxr,) = torch.autograd.grad(out, xd, gout.to(DEV))
    _check_grad(gxr, L.lif_reverse(x.float(), gout, forward_dtype=torch.float32),
                torch.bfloat16, "residual grad_x 216M shape")


# Exact float32 threshold ties: the pre-spike membrane equals fp32(threshold),
# so h - threshold == 0 and the step fires (language.py:834-836).  The kernels
# must fire there as the float32 loop does, and their gradients must follow
# the float32 spike pattern on every step after the tie.
TIE_CASES = {
    # B=64 T=1024 C=512 fp32, tau 2, threshold 1.3, slope 1.5, with x = 1.3
    # planted every seventh step (after a reset, h = x exactly).
    "fp32_full_size": dict(shape=(64, 1024, 512), dtype=torch.float32, tau=2.0, threshold=1.3,
                           slope=1.5, scale=1.5, plant=1.3),
    # B=64 T=33 C=256 bf16, tau 3, threshold 1, slope 1.5: 1.0 is a bf16 value,
    # so after a reset the membrane hits the threshold exactly wherever x = 1.
    "bf16_short": dict(shape=(64, 33, 256), dtype=torch.bfloat16, tau=3.0, threshold=1.0,
                       slope=1.5, scale=1.5, plant=1.0),
}


@pytest.mark.parametrize("case", list(TIE_CASES))
def test_exact_threshold_ties(case):
    p = TIE_CASES[case]
    b, t, c = p["shape"]
    dtype = p["dtype"]
    print(f"lif ties {case}", flush=True)
    x, gs = _inputs(b, t, c, dtype, seed=31, scale=p["scale"])
    x[:, 3::7] = p["plant"]
    h, s_ref = L.lif_membranes(x.float(), p["tau"], p["threshold"], 0.0, p["slope"],
                               dtype=torch.float32)
    thr32 = float(torch.tensor(p["threshold"], dtype=torch.float32))
    ties = int((h == thr32).sum())
    assert ties > 0, "the inputs must hold exact ties"
    spikes, gx = _run(x, gs, tau=p["tau"], threshold=p["threshold"], reset=0.0, slope=p["slope"])
    assert torch.equal(spikes.float(), s_ref), f"spikes differ ({ties} ties)"
    ref = L.lif_reverse(x.float(), gs.float(), p["tau"], p["threshold"], 0.0, p["slope"],
                        forward_dtype=torch.float32)
    _check_grad(gx, ref, dtype, f"grad_x at {ties} exact ties")
