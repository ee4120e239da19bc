"""ZDF SVF bank on the GPU against the oracle (dgen_oracle_svf_fwd / _step):
the linear bank's chunked forward and the saturating bank's per-lane forward,
the BPTT gradient to (base, res, kSat) and d loss / d x, at 256 lanes x 2^18
frames (SvfConfig), and the streaming process path (any split of a signal
into calls gives the same samples).  fp32 recurrences: the HIP results must
stay within 2x the fp32 oracle's distance from the fp64 oracle.  Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import SvfConfig
from dgen_hip.programs import SvfSession, stream_svf_program
from dgen_hip.runtime import HIPLazyRuntime


pytestmark = pytest.mark.gpu


def oracle_args(cfg, params):
    P = len(params) // cfg.B
    p = params.reshape(P, cfg.B)
    return dict(base=p[0], res=p[1], ks=p[2] if P == 3 else None, m=cfg.modulation(), env=cfg.envelope(), sr=cfg.sr)


@pytest.fixture(scope="module", params=[False, True], ids=["linear", "saturating"])
def svf_run(request):
    cfg = SvfConfig(saturating=request.param)
    print(f"SVF bank B={cfg.B} T={cfg.T} saturating={cfg.saturating}", flush=True)
    s = SvfSession(cfg, optimizer=False)
    try:
        s.step()
        out = dict(cfg=cfg, x=s.x, target=s.target, y=s.rt.read("y").reshape(cfg.T, cfg.B), loss=s.loss(),
                   grads=s.rt.read("grads").astype(np.float64), params=s.params0)
    finally:
        s.close()
    return out


def test_target_bank_matches_the_oracle(svf_run):
    cfg = svf_run["cfg"]
    a = oracle_args(cfg, cfg.target_params())
    a["ks"] = None
    ref32 = O.svf_fwd(svf_run["x"], **a)
    ref64 = O.svf_fwd(svf_run["x"], **a, prec="f64")
    e_hip, e_o32 = np.abs(svf_run["target"] - ref64).max(), np.abs(ref32 - ref64).max()
    print(f"target bank: max|y - fp64| HIP {e_hip:.3e}, fp32 oracle {e_o32:.3e}")
    assert e_hip <= 2.0 * e_o32 + 1e-6


def test_forward_loss_and_gradient_match_the_oracle(svf_run):
    cfg, x, tgt = svf_run["cfg"], svf_run["x"], svf_run["target"]
    a = oracle_args(cfg, svf_run["params"])
    l64, g64, y64, _ = O.svf_step(x, tgt=tgt, want_y=True, **a)
    l32, g32, y32, _ = O.svf_step(x, tgt=tgt, want_y=True, prec="f32", **a)
    y = svf_run["y"]
    e_hip, e_o32 = np.abs(y - y64).max(), np.abs(y32 - y64).max()
    print(f"y: max|y - fp64| HIP {e_hip:.3e}, fp32 oracle {e_o32:.3e} (max |y| {np.abs(y64).max():.3f})")
    assert e_hip <= 2.0 * e_o32 + 1e-6
    loss = svf_run["loss"]
    print(f"loss HIP {loss:.8e}, fp64 oracle {l64:.8e}, fp32 oracle {l32:.8e}")
    assert abs(loss - l64) <= 2.0 * abs(l32 - l64) + 1e-5 * abs(l64)
    g = svf_run["grads"]
    P = cfg.P
    for r, name in enumerate(["base", "res", "kSat"][:P]):
        sl = slice(r * cfg.B, (r + 1) * cfg.B)
        nrm = np.linalg.norm(g64[sl])
        eh, eo = np.linalg.norm(g[sl] - g64[sl]) / nrm, np.linalg.norm(g32[sl] - g64[sl]) / nrm
        print(f"d/d {name}: rel L2 vs fp64 HIP {eh:.3e}, fp32 oracle {eo:.3e}")
        assert eh <= 2.0 * eo + 1e-5


@pytest.mark.parametrize("B,T,chunk", [(64, 4096, 256), (70, 3001, 7), (256, 1 << 18, 256)])
def test_fused_adjoint_summaries_equal_the_reverse_pass(B, T, chunk):
    """Linear bank: the forward replay's prefix-product adjoint summaries and
    the separate reverse pass compose the same affine chunk maps: equal to
    fp64 rounding, the gradients to fp32 rounding."""
    cfg = SvfConfig(B=B, T=T, saturating=False)
    print(f"case B={B} T={T} chunk={chunk}", flush=True)
    target = None
    out = {}
    for fused in (True, False):
        s = SvfSession(cfg, optimizer=False, chunk=chunk, target=target, fuse_adjoint=fused)
        target = s.target
        try:
            s.step()
            out[fused] = (s.rt.read("adj_summary").view(np.float64), s.rt.read("grads"), s.loss())
        finally:
            s.close()
    (a1, g1, l1), (a0, g0, l0) = out[True], out[False]
    assert abs(l1 - l0) <= 1e-6 * abs(l0)
    scale = np.abs(a0).max()
    print(f"summary max diff {np.abs(a1 - a0).max():.3e} (scale {scale:.3e})")
    np.testing.assert_allclose(a1, a0, rtol=0, atol=1e-12 * scale)
    np.testing.assert_allclose(g1, g0, rtol=1e-5, atol=1e-6 * np.abs(g0).max())


def test_input_gradient_matches_the_oracle():
    for sat in (False, True):
        cfg = SvfConfig(B=64, T=1 << 14, saturating=sat)
        s = SvfSession(cfg, optimizer=False, xbar=True)
        try:
            s.step()
            xb = s.rt.read("xbar").reshape(cfg.T, cfg.B).astype(np.float64)
        finally:
            s.close()
        a = oracle_args(cfg, cfg.params())
        _, _, _, xb64 = O.svf_step(s.x, tgt=s.target, want_xbar=True, grad=False, **a)
        _, _, _, xb32 = O.svf_step(s.x, tgt=s.target, want_xbar=True, grad=False, prec="f32", **a)
        nrm = np.linalg.norm(xb64)
        eh, eo = np.linalg.norm(xb - xb64) / nrm, np.linalg.norm(xb32 - xb64) / nrm
        print(f"saturating={sat}: d loss / d x rel L2 vs fp64 HIP {eh:.3e}, fp32 oracle {eo:.3e}")
        assert eh <= 2.0 * eo + 1e-6


def test_streaming_calls_carry_the_cells():
    cfg = SvfConfig(B=64, T=1 << 15, saturating=True)
    prog = stream_svf_program(cfg)
    x, m, env, prm = cfg.inputs(), cfg.modulation(), cfg.envelope(), cfg.params()
    rt = HIPLazyRuntime(prog, 0)
    try:
        rt.write("params", prm)
        rt.setProcessPorts(*prog.meta["ports"])

        def calls(sizes):
            out, n0 = [], 0
            for i, n in enumerate(sizes):
                ins = [x[n0:n0 + n, k] for k in range(cfg.B)] + [m[n0:n0 + n], env[n0:n0 + n]]
                out.append(rt.process(ins, n, reset=i == 0).T)
                n0 += n
            return np.concatenate(out)

        one = calls([cfg.T])
        for sizes in ([8192] * 4, [1, 4095, 20000, 8672]):
            np.testing.assert_array_equal(calls(sizes), one)
    finally:
        rt.close()
    a = oracle_args(cfg, prm)
    st = np.zeros((2, cfg.B), np.float32)
    ref = np.concatenate([O.svf_fwd(x[:9000], **{**a, "m": a["m"][:9000], "env": a["env"][:9000]}, state=st),
                          O.svf_fwd(x[9000:], **{**a, "m": a["m"][9000:], "env": a["env"][9000:]}, state=st)])
    ref64 = O.svf_fwd(x, **a, prec="f64")
    print(f"stream: max|y - fp32 oracle| {np.abs(one - ref).max():.3e}, HIP vs fp64 {np.abs(one - ref64).max():.3e}, "
          f"fp32 oracle vs fp64 {np.abs(ref - ref64).max():.3e}")
    assert np.abs(one - ref64).max() <= 2.0 * np.abs(ref - ref64).max() + 1e-6


def test_training_forward_through_lds_tiles_equals_the_per_frame_kernel():
    """The saturating training forward (the LDS-tiled lane loop: 32-frame
    tiles by 16-byte copies) and the streaming kernel (per-frame loads and
    stores, coefficients evaluated in the loop) give the same y bit for bit
    on the same input and parameters."""
    cfg = SvfConfig(B=128, T=1 << 14, saturating=True)
    s = SvfSession(cfg, optimizer=False)
    try:
        s.step()
        y = s.rt.read("y").reshape(cfg.T, cfg.B)
        labels = [op.label for op in s.program.ops]
    finally:
        s.close()
    prog = stream_svf_program(cfg)
    x, m, env = cfg.inputs(), cfg.modulation(), cfg.envelope()
    rt = HIPLazyRuntime(prog, 0)
    try:
        rt.write("params", cfg.params())
        rt.setProcessPorts(*prog.meta["ports"])
        one = rt.process([x[:, k] for k in range(cfg.B)] + [m, env], cfg.T, reset=True).T
    finally:
        rt.close()
    assert "svf_seq" in labels
    np.testing.assert_array_equal(y, one)


@pytest.mark.parametrize("B,T,chunk", [(64, 4096 + 32, 256), (128, 48000, 256)])
def test_saturating_training_loss_covers_a_ragged_last_chunk(B, T, chunk):
    """The saturating training forward on LDS tiles with T not a multiple of
    the chunk length: the last chunk's loss partial (T mod L frames) is
    written, so the loss is the whole signal's (against the oracle) and the
    gradient is unchanged."""
    cfg = SvfConfig(B=B, T=T, saturating=True)
    print(f"case B={B} T={T} chunk={chunk}", flush=True)
    s = SvfSession(cfg, optimizer=False, chunk=chunk)
    try:
        s.step()
        loss, labels = s.loss(), [op.label for op in s.program.ops]
        g = s.rt.read("grads").astype(np.float64)
    finally:
        s.close()
    assert "svf_seq" in labels
    a = oracle_args(cfg, s.params0)
    l64, g64, _, _ = O.svf_step(s.x, tgt=s.target, **a)
    l32, _, _, _ = O.svf_step(s.x, tgt=s.target, prec="f32", **a)
    print(f"loss HIP {loss:.8e}, fp64 oracle {l64:.8e}, fp32 oracle {l32:.8e}")
    assert abs(loss - l64) <= 2.0 * abs(l32 - l64) + 1e-5 * abs(l64)
    assert np.linalg.norm(g - g64) <= 1e-4 * np.linalg.norm(g64)
