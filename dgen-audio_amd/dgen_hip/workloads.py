"""Synthetic, seeded inputs for the five benchmark workloads.

All randomness comes from SplitMix64, the generator the reference's
HarmonicE2E example uses (Examples/HarmonicE2E/Config.swift:245-259), so every
array here is reproducible bit-for-bit on any host.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

_M64 = (1 << 64) - 1


class SplitMix64:
    """SplitMix64 stream; seed 0 is replaced by the golden-ratio increment
    (Examples/HarmonicE2E/Config.swift:248-258)."""

    def __init__(self, seed: int):
        self.state = 0x9E3779B97F4A7C15 if seed == 0 else seed & _M64

    def next(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & _M64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
        return z ^ (z >> 31)

    def next_array(self, n: int) -> np.ndarray:
        """n raw uint64 draws, vectorised (identical to n calls of next())."""
        inc = np.uint64(0x9E3779B97F4A7C15)
        with np.errstate(over="ignore"):
            st = np.uint64(self.state) + inc * np.arange(1, n + 1, dtype=np.uint64)
            z = st
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            z = z ^ (z >> np.uint64(31))
        self.state = int(st[-1]) if n else self.state
        return z

    def uniform(self, n: int) -> np.ndarray:
        """U[0,1) doubles from the top 53 bits."""
        return (self.next_array(n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))

    def normal(self, n: int) -> np.ndarray:
        """Box-Muller N(0,1) doubles."""
        m = (n + 1) // 2
        u1 = np.maximum(self.uniform(m), 1e-300)
        u2 = self.uniform(m)
        r = np.sqrt(-2.0 * np.log(u1))
        return np.concatenate([r * np.cos(2 * math.pi * u2), r * np.sin(2 * math.pi * u2)])[:n]


def reference_random_array(rng: SplitMix64, count: int, scale: float) -> np.ndarray:
    """HarmonicDecoderModel.randomArray (Examples/HarmonicE2E/Model.swift:141-151):
    r = Float(next() & 0xFFFF) / Float(UInt16.max); w = (r*2 - 1) * scale."""
    raw = (rng.next_array(count) & np.uint64(0xFFFF)).astype(np.float32)
    r = raw / np.float32(65535.0)
    return ((r * np.float32(2.0) - np.float32(1.0)) * np.float32(scale)).astype(np.float32)


# ---------------------------------------------------------------- config 1
@dataclass
class OscBankConfig:
    n_osc: int = 16
    f_base: float = 220.0
    sr: float = 44100.0
    pole: float = 0.9
    frames: int = 65536
    seed: int = 1

    def inputs(self):
        freqs = (np.arange(1, self.n_osc + 1, dtype=np.float32) * np.float32(self.f_base)).astype(np.float32)
        a = SplitMix64(self.seed).uniform(self.n_osc).astype(np.float32)
        amps = (a / a.sum(dtype=np.float32)).astype(np.float32)
        return freqs, amps


# ---------------------------------------------------------------- config 3
@dataclass
class HarmonicConfig:
    """Batched DDSP harmonic + FIR-noise synth with MLP decoder and MSS loss."""
    B: int = 32
    T: int = 64000
    sr: float = 16000.0
    K: int = 60
    NF: int = 65
    control_hop: int = 64
    din: int = 2
    hidden: int = 512
    layers: int = 3
    fft_sizes: tuple = (2048, 1024, 512, 256, 128, 64)
    hop_div: int = 4
    w_lin: float = 1.0
    w_log: float = 0.5
    # spectralLossFFT options of the two terms (HigherOps.swift:49-65,
    # Functions.swift:870-910): lossMode "l1" (the trainer's) or "l2" (the
    # API default) per term, useSmoothLogMagnitude for the log term,
    # useHannWindow; and the trainer's mseLossWeight (Trainer.swift:547-551)
    loss_lin: str = "l1"
    loss_log: str = "l1"
    smooth_log: bool = False
    hann: bool = True
    w_mse: float = 0.0
    min_f0: float = 50.0
    max_f0: float = 1000.0
    hscale: float = 1.0
    nscale: float = 1.0
    data_seed: int = 3
    weight_seed: int = 5
    target_seed: int = 4
    lr: float = 1e-3
    # products of the MLP GEMMs: "split-bf16" (each fp32 operand split into
    # three bfloat16 parts, six partial products accumulated in fp32: as
    # accurate as fp32 products, on the bf16 matrix cores) or "fp32" (the
    # fp32 matrix cores)
    gemm_products: str = "split-bf16"

    @property
    def F(self) -> int:
        return max(1, self.T // self.control_hop)

    @property
    def NC(self) -> int:
        return self.K + 2 + self.NF

    @property
    def mss_mode(self) -> int:
        """Loss-mode bits of the multi-scale loss: 1 magnitude term L2, 2 log
        term L2, 4 smooth log magnitude, 8 rectangular window."""
        for name, v in (("loss_lin", self.loss_lin), ("loss_log", self.loss_log)):
            if v not in ("l1", "l2"):
                raise ValueError(f"{name} {v!r}: 'l1' or 'l2'")
        return ((1 if self.loss_lin == "l2" else 0) | (2 if self.loss_log == "l2" else 0)
                | (4 if self.smooth_log else 0) | (0 if self.hann else 8))

    @property
    def M(self) -> int:
        return self.B * self.F

    @property
    def ldc(self) -> int:
        """Padded stride of the control rows (Z, ctrl, dctrl, dZ): 128 for
        up to 128 columns, else NC rounded up to 64."""
        return 128 if self.NC <= 128 else (self.NC + 63) // 64 * 64

    def param_count(self) -> int:
        n, fan = 0, self.din
        for _ in range(self.layers):
            n += fan * self.hidden + self.hidden
            fan = self.hidden
        return n + self.hidden * self.NC + self.NC

    def weights(self, seed: int | None = None) -> np.ndarray:
        """Parameter blob in the order W1 b1 ... WL bL Wh bh; head columns are
        W_harm | W_gain | W_noise | W_noiseFilter.  Initialisation follows
        HarmonicDecoderModel.init (Examples/HarmonicE2E/Model.swift:36-83),
        drawing the tensors in the reference's order."""
        rng = SplitMix64(self.weight_seed if seed is None else seed)
        parts = []
        fan = self.din
        for _ in range(self.layers):
            scale = np.float32(math.sqrt(2.0 / fan) * 0.5)
            parts.append(reference_random_array(rng, fan * self.hidden, scale))
            parts.append(np.zeros(self.hidden, np.float32))
            fan = self.hidden
        H, K, NF = self.hidden, self.K, self.NF
        w_harm = reference_random_array(rng, H * K, 0.06).reshape(H, K)
        w_gain = reference_random_array(rng, H, 0.05).reshape(H, 1)
        w_noise = reference_random_array(rng, H, 0.05).reshape(H, 1)
        w_nf = reference_random_array(rng, H * NF, 0.05).reshape(H, NF)
        parts.append(np.concatenate([w_harm, w_gain, w_noise, w_nf], axis=1).reshape(-1))
        bh = np.zeros(self.NC, np.float32)
        bh[K + 1] = -3.0  # b_noise init (Model.swift:77)
        parts.append(bh)
        return np.concatenate(parts).astype(np.float32)

    def data(self):
        """f0 [F][B] (Hz), uv [F][B], features X [B*F][din] (row = b*F + f).

        f0: log-uniform start in [60, 1000] Hz, then a Gaussian log-domain
        random walk (sigma 0.01 per control frame); loudness ~ U[0,1].
        Features follow makeConditioningData (Examples/HarmonicE2E/Trainer.swift:588-616):
        f0_norm = (log(max(f0,minF0)) - log(minF0)) / (log(maxF0) - log(minF0)),
        loudness as given; uv = 1 (voiced)."""
        rng = SplitMix64(self.data_seed)
        B, F = self.B, self.F
        start = math.log(60.0) + rng.uniform(B) * (math.log(1000.0) - math.log(60.0))
        walk = np.cumsum(rng.normal(F * B).reshape(F, B) * 0.01, axis=0)
        walk -= walk[0:1]
        f0 = np.exp(start[None, :] + walk).astype(np.float32)
        loud = rng.uniform(F * B).reshape(F, B).astype(np.float32)
        uv = np.ones((F, B), np.float32)
        lo, hi = math.log(self.min_f0), math.log(max(self.max_f0, self.min_f0 + 1))
        f0n = ((np.log(np.maximum(f0.astype(np.float64), self.min_f0)) - lo) / max(1e-6, hi - lo)).astype(np.float32)
        X = np.zeros((B * F, self.din), np.float32)
        X[:, 0] = f0n.T.reshape(-1)
        if self.din > 1:
            X[:, 1] = loud.T.reshape(-1)
        if self.din > 2:
            X[:, 2] = uv.T.reshape(-1)
        return f0, uv, X


# ---------------------------------------------------------------- config 4
@dataclass
class BiquadConfig:
    """Tensor biquad bank with BPTT: B lanes x T samples of U[-1,1] noise
    through an RBJ low-pass whose cutoff base[k] * m[n] follows a geometric
    f_lo -> f_hi sweep driven by a sine LFO; loss = sum (y - y_target)^2
    against a fixed (tgt_fc, tgt_Q) bank; gradients w.r.t. base and Q."""
    B: int = 256
    T: int = 1 << 18
    sr: float = 44100.0
    lfo_hz: float = 2.0
    f_lo: float = 200.0
    f_hi: float = 4000.0
    base0: float = 200.0
    Q0: float = 0.707
    tgt_fc: float = 1000.0
    tgt_Q: float = 0.707
    seed: int = 40
    lr: float = 1e-3

    def inputs(self) -> np.ndarray:
        """x [T][B]: lane k is U[-1,1] drawn from SplitMix64(seed + k)."""
        x = np.empty((self.T, self.B), np.float32)
        for k in range(self.B):
            x[:, k] = (SplitMix64(self.seed + k).uniform(self.T) * 2.0 - 1.0).astype(np.float32)
        return x

    def modulation(self) -> np.ndarray:
        """m [T] in fp32, so that base[k] * m[n] sweeps geometrically between
        base*1 and base*(f_hi/f_lo): the LFO is the deterministic phasor
        frac((lfo/sr) * n) (Sources/DGen/Emit+State.swift:382-386) through
        sin(2 pi p), mapped to m = (f_hi/f_lo)^(0.5 + 0.5 sin)."""
        n = np.arange(self.T, dtype=np.float32)
        r = np.float32(self.lfo_hz / self.sr) * n
        ph = (r - np.floor(r)).astype(np.float32)
        s = np.sin(np.float32(2.0 * math.pi) * ph, dtype=np.float32)
        e = (np.float32(0.5) + np.float32(0.5) * s).astype(np.float32)
        return np.exp2(np.float32(math.log2(self.f_hi / self.f_lo)) * e, dtype=np.float32).astype(np.float32)

    def params(self) -> np.ndarray:
        """Parameter blob [2][B] = base | Q."""
        return np.concatenate([np.full(self.B, self.base0, np.float32), np.full(self.B, self.Q0, np.float32)])

    def target_params(self) -> np.ndarray:
        return np.concatenate([np.full(self.B, self.tgt_fc, np.float32), np.full(self.B, self.tgt_Q, np.float32)])


# ------------------------------------------------------ ZDF SVF bank (BPTT)
@dataclass
class SvfConfig:
    """Two-cell ZDF SVF low-pass bank with BPTT (the MonologueVoice filter of
    Tests/DGenLazyTests/SVFBPTTScratchTests.swift:21-34, one per lane): B
    lanes x T samples of U[-1,1] noise; the cutoff of lane k at frame n is
    clip(base[k] * m[n] + env[n], 20, 20000) with m the config-4 LFO sweep
    and env = env_depth * exp(-t / env_tau) (the reference's cutoff envelope,
    :56-63); kDamp = 1 / res[k]; with ``saturating`` each lane also learns
    its kSat.  Loss = sum (y - y_target)^2 against a linear bank with
    (tgt_fc, tgt_res); gradients w.r.t. base, res (and kSat)."""
    B: int = 256
    T: int = 1 << 18
    sr: float = 44100.0
    lfo_hz: float = 2.0
    f_lo: float = 200.0
    f_hi: float = 4000.0
    env_depth: float = 900.0
    env_tau: float = 0.15
    base_lo: float = 150.0
    base_hi: float = 2500.0
    res_lo: float = 0.6
    res_hi: float = 3.0
    ks_hi: float = 2.0
    tgt_fc: float = 1000.0
    tgt_res: float = 1.2
    saturating: bool = False
    seed: int = 40
    lr: float = 1e-3

    @property
    def P(self) -> int:
        """Parameters per lane: base, res (, kSat)."""
        return 3 if self.saturating else 2

    def inputs(self) -> np.ndarray:
        """x [T][B]: lane k is U[-1,1] drawn from SplitMix64(seed + k)."""
        x = np.empty((self.T, self.B), np.float32)
        for k in range(self.B):
            x[:, k] = (SplitMix64(self.seed + k).uniform(self.T) * 2.0 - 1.0).astype(np.float32)
        return x

    def modulation(self) -> np.ndarray:
        """m [T]: the config-4 geometric LFO sweep (f_hi/f_lo)^(0.5 + 0.5 sin)."""
        return BiquadConfig(T=self.T, sr=self.sr, lfo_hz=self.lfo_hz, f_lo=self.f_lo, f_hi=self.f_hi).modulation()

    def envelope(self) -> np.ndarray:
        """env [T] in fp32: env_depth * exp(-t / env_tau), t = n / sr."""
        t = (np.arange(self.T, dtype=np.float64) / self.sr).astype(np.float32)
        return (np.float32(self.env_depth) * np.exp(-t / np.float32(self.env_tau))).astype(np.float32)

    def params(self) -> np.ndarray:
        """Parameter blob [P][B] = base | res (| kSat), spread over the lanes."""
        u = np.linspace(0.0, 1.0, self.B)
        base = self.base_lo * (self.base_hi / self.base_lo) ** u
        res = self.res_lo + (self.res_hi - self.res_lo) * u[::-1]
        rows = [base, res] + ([self.ks_hi * u] if self.saturating else [])
        return np.concatenate(rows).astype(np.float32)

    def target_params(self) -> np.ndarray:
        """The linear target bank's [2][B] = tgt_fc | tgt_res."""
        return np.concatenate([np.full(self.B, self.tgt_fc, np.float32), np.full(self.B, self.tgt_res, np.float32)])


# ------------------------------------------------- temporal gradient (a21)
@dataclass
class SweptPhasorConfig:
    """A bank of E swept phasors with learnable sweep rates: the graph of
    Tests/DGenLazyTests/TemporalGradientTests.swift:24-60 per lane, f[n] =
    base + slope[e] * time[n] with time = accum(1/sr), phase =
    statefulPhasor(f, reset), loss = sum (phase - target)^2, or with
    ``smooth`` sum (sin(2 pi phase) - target)^2 (continuous across the
    phase's wraps, so finite differences of long runs are meaningful);
    resets from frame reset_from on (-1: none)."""
    E: int = 256
    T: int = 1 << 16
    sr: float = 44100.0
    base: float = 80.0
    target: float = 0.08
    reset_from: int = -1
    smooth: bool = True
    slope_lo: float = 600.0
    slope_hi: float = 24000.0
    lr: float = 1e-3

    def slopes(self) -> np.ndarray:
        """Geometric sweep rates slope_lo .. slope_hi across the lanes."""
        if self.E == 1:
            return np.array([self.slope_lo], np.float32)
        r = np.arange(self.E, dtype=np.float64) / (self.E - 1)
        return (self.slope_lo * (self.slope_hi / self.slope_lo) ** r).astype(np.float32)

    def reset(self) -> np.ndarray:
        n = np.arange(self.T)
        return ((n >= self.reset_from) & (self.reset_from >= 0)).astype(np.float32)


# ---------------------------------------------------------------- config 2
@dataclass
class StftConfig:
    """Hop-gated STFT round trip: S signals x [S][T] of N(0, sigma^2) noise,
    buffer N / hop H, periodic Hann (DGenLazy hann(N)), FFT, per-bin gains
    g[N/2+1] (init 1.0) on the one-sided spectrum, IFFT, overlapAdd; loss
    sum (y - x)^2 / T against the raw input; gradient w.r.t. g."""
    S: int = 8
    T: int = 1 << 20
    N: int = 1024
    H: int = 256
    sigma: float = 0.5
    seed: int = 20
    lr: float = 1e-3

    @property
    def bins(self) -> int:
        return self.N // 2 + 1

    def inputs(self) -> np.ndarray:
        """x [S][T]: signal s is N(0, sigma^2) from SplitMix64(seed + s)."""
        x = np.empty((self.S, self.T), np.float32)
        for s in range(self.S):
            x[s] = (SplitMix64(self.seed + s).normal(self.T) * self.sigma).astype(np.float32)
        return x

    def window(self) -> np.ndarray:
        """hann(N) of Sources/DGenLazy/SpectralTensorOps.swift:42-49, in fp32:
        scale = 2*Float.pi/Float(N); w[i] = 0.5 - 0.5*cos(scale*Float(i))."""
        scale = np.float32(np.float32(2.0) * np.float32(math.pi)) / np.float32(self.N)
        arg = (scale * np.arange(self.N, dtype=np.float32)).astype(np.float32)
        return (np.float32(0.5) - np.float32(0.5) * np.cos(arg, dtype=np.float32)).astype(np.float32)

    def gains(self) -> np.ndarray:
        return np.ones(self.bins, np.float32)


# ---------------------------------------------------------------- config 5
@dataclass
class MembraneConfig:
    """2D membrane: R x C grid, u_{t+1} = 2u_t - u_{t-1} + c2 L(u_t)
    - d (u_t - u_{t-1}) with the 3x3 zero-padded Laplacian, Gaussian-bump
    initial displacement (u_{-1} = u_0), T steps, pickup out[n] = u_{n+1}[p];
    loss sum (out - out_target)^2 against the same model with (tgt_c2, tgt_d);
    gradients w.r.t. (c2, d)."""
    R: int = 512
    C: int = 512
    T: int = 4800
    c2: float = 0.2
    d: float = 0.001
    tgt_c2: float = 0.25
    tgt_d: float = 0.002
    sigma: float = 4.0
    seed: int = 50
    lr: float = 1e-3

    @property
    def pickup(self) -> tuple:
        return (self.R // 2, (self.C * 300) // 512)

    def bump(self) -> np.ndarray:
        """u_0: unit Gaussian (sigma cells) centred at a SplitMix64(seed)
        position at least R/8 (C/8) cells inside the edges."""
        rng = SplitMix64(self.seed)
        my, mx = self.R // 8, self.C // 8
        cy = my + int(rng.next() % max(1, self.R - 2 * my))
        cx = mx + int(rng.next() % max(1, self.C - 2 * mx))
        y = np.arange(self.R, dtype=np.float64)[:, None]
        x = np.arange(self.C, dtype=np.float64)[None, :]
        r2 = (y - cy) ** 2 + (x - cx) ** 2
        return np.exp(-r2 / (2.0 * self.sigma ** 2)).astype(np.float32)

    def params(self) -> np.ndarray:
        return np.array([self.c2, self.d], np.float32)

    def target_params(self) -> np.ndarray:
        return np.array([self.tgt_c2, self.tgt_d], np.float32)
