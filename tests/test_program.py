"""Host-side schedule construction: cell layout, operand shapes and the cost
model the roofline figures come from.  CPU only."""
import numpy as np
import pytest

from dgen_hip import HarmonicConfig
from dgen_hip import runtime as R
from dgen_hip.program import ALIGN, Program
from dgen_hip.programs import harmonic_program, oscbank_program
from dgen_hip.roofline import roof_seconds, step_roof_ms
from dgen_hip.workloads import OscBankConfig, SplitMix64


def test_cells_are_aligned_and_disjoint():
    p = harmonic_program(HarmonicConfig())
    cells = sorted(p.cells.values(), key=lambda c: c.off)
    for a, b in zip(cells, cells[1:]):
        assert a.off % ALIGN == 0 and a.off + a.n <= b.off
    assert cells[-1].off + cells[-1].n == p.size


def test_op_operands_lie_in_cells():
    p = harmonic_program(HarmonicConfig(B=4, T=4096))
    starts = {c.off: c for c in p.cells.values()}
    for op in p.ops:
        # every cell-typed operand the schedule passes starts a cell
        for a in op.arg[:3]:
            if a > 0 and a in starts:
                assert starts[a].off + starts[a].n <= p.size


def test_train_schedule_order():
    labels = [op.label for op in harmonic_program(HarmonicConfig()).ops if not op.flags & R.OP_STATIC]
    assert labels.index("phasor_carry") < labels.index("synth_fwd") < labels.index("spectral_mss")
    assert labels.index("spectral_mss") < labels.index("synth_bwd") < labels.index("synth_bwd_reduce")
    assert labels[-1] == "adam"


@pytest.mark.parametrize("products,bound,roof", [("fp32", "mfma", (0.5, 2.0)), ("split-bf16", "mfma_x6", (0.2, 1.0))])
def test_roofline_model_config3(products, bound, roof):
    p = harmonic_program(HarmonicConfig(gemm_products=products))
    gemm = [op for op in p.ops if op.bound in ("mfma", "mfma_x6")]
    assert all(op.bound == bound for op in gemm)
    flops = sum(op.flops for op in gemm)
    # 3 x 512 MLP over 32000 rows: forward + two backward GEMMs per layer
    assert abs(flops - 2 * 32000 * (2 * 512 * 512 * 3 + 512 * 127 * 3)) < 1e6
    assert roof[0] < step_roof_ms(p) < roof[1]
    assert all(roof_seconds(op) >= 0 for op in p.ops)
    # the split-bf16 GEMM roof: six bf16 partial products per fp32 product
    if bound == "mfma_x6":
        op = next(op for op in gemm if op.label == "mlp_l2")
        assert roof_seconds(op) == pytest.approx(op.flops * 6 / 2.5e15)


def test_invalid_configs_raise():
    with pytest.raises(ValueError, match="harmonics"):
        harmonic_program(HarmonicConfig(K=257))
    with pytest.raises(ValueError, match="exceeds 512"):
        harmonic_program(HarmonicConfig(K=256, NF=255))
    with pytest.raises(ValueError):
        harmonic_program(HarmonicConfig(fft_sizes=(4096,)))
    with pytest.raises(ValueError):
        Program().alloc("x", 0)


def test_wide_harmonic_programs_use_a_wider_row_stride():
    # one group and <= 128 columns keep the 128 stride; beyond, NC rounded up to 64
    for (K, NF, ldc) in [(60, 65, 128), (64, 62, 128), (65, 63, 192), (100, 100, 256), (256, 254, 512)]:
        cfg = HarmonicConfig(B=2, T=6400, K=K, NF=NF, hidden=64)
        assert cfg.ldc == ldc
        p = harmonic_program(cfg)
        assert p.cells["ctrl"].n == cfg.M * ldc and p.cells["dZ"].n == cfg.M * ldc
        assert p.cells["checkpoints"].n == ((cfg.T + 63) // 64) * cfg.B * K


def test_splitmix_matches_reference_sequence():
    # SplitMix64 with seed 0 replaced by the golden-ratio increment
    # (Examples/HarmonicE2E/Config.swift:245-259); vector and scalar agree
    a, b = SplitMix64(5), SplitMix64(5)
    v = a.next_array(100)
    s = np.array([b.next() for _ in range(100)], np.uint64)
    np.testing.assert_array_equal(v, s)
    # first output of seed 1 (the published SplitMix64 test value)
    assert SplitMix64(1).next() == 0x910A2DEC89025CC1


def test_weights_follow_reference_init():
    cfg = HarmonicConfig()
    w = cfg.weights()
    assert w.dtype == np.float32 and len(w) == cfg.param_count()
    # b_noise starts at -3 (Model.swift:77), every other bias at 0
    bh = w[-cfg.NC:]
    assert bh[cfg.K + 1] == -3.0 and np.count_nonzero(bh) == 1
    # trunk layer 1 scale sqrt(2/fan)*0.5
    w1 = w[:cfg.din * cfg.hidden]
    assert np.abs(w1).max() <= np.sqrt(2 / cfg.din) * 0.5 + 1e-6


def test_oscbank_program():
    cfg = OscBankConfig()
    p = oscbank_program(cfg)
    assert p.output_cell == "out" and p.cells["out"].n == cfg.frames


def test_oscbank_inputs_follow_config():
    freqs, amps = OscBankConfig().inputs()
    np.testing.assert_array_equal(freqs, (np.arange(1, 17) * 220.0).astype(np.float32))
    assert abs(float(amps.sum()) - 1.0) < 1e-6
