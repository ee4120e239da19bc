"""On-disk formats: WAV I/O (Sources/DGenLazy/AudioFile.swift), model
checkpoints (Examples/HarmonicE2E/Checkpoint.swift, Model.swift:122-141;
Examples/DDSPE2E/Checkpoint.swift) and the HarmonicE2E dataset cache
(Examples/HarmonicE2E/Dataset.swift, Features.swift, Trainer.swift:589-617).
The WAV cases include every case of Tests/DGenLazyTests/WAVParsingTests.swift;
PCM decoding is cross-checked with Python's own ``wave`` module.  CPU only."""
import io
import json
import math
import os
import struct
import wave

import numpy as np
import pytest

from dgen_hip import HarmonicConfig, SplitMix64
from dgen_hip import audiofile as A
from dgen_hip import checkpoint as C
from dgen_hip import dataset as D
from dgen_hip.workloads import reference_random_array


# ------------------------------------------------------------------- WAV
def make_wav(fmt, channels, rate, bits, payload, fmt_size=16, extra=None, declared=None):
    """WAVParsingTests.makeWAV: full control over the fmt chunk size, the
    declared data size and an ancillary chunk between fmt and data."""
    align = channels * bits // 8
    f = struct.pack("<HHIIHH", fmt, channels, rate, rate * align, align, bits).ljust(fmt_size, b"\0")
    body = b"WAVE" + b"fmt " + struct.pack("<I", fmt_size) + f
    if extra:
        body += extra[0] + struct.pack("<I", len(extra[1])) + extra[1]
    body += b"data" + struct.pack("<I", len(payload) if declared is None else declared) + payload
    return b"RIFF" + struct.pack("<I", len(body)) + body


def f32(values):
    return np.array(values, "<f4").tobytes()


def test_partial_frame_is_dropped():
    s, _ = A.parse_wav(make_wav(1, 2, 8000, 16, b"\x01" * 6))
    assert s.size == 1


def test_no_complete_frame_raises():
    with pytest.raises(A.AudioFileError):
        A.parse_wav(make_wav(1, 2, 8000, 16, b"\x01" * 2))


def test_declared_data_size_beyond_the_file_is_clamped():
    s, rate = A.parse_wav(make_wav(3, 1, 8000, 32, f32([0.25, -0.5, 0.75]), declared=0xFFFFFFFF))
    assert rate == 8000.0 and s.tolist() == [0.25, -0.5, 0.75]


def test_truncated_fmt_chunk_raises():
    with pytest.raises(A.AudioFileError):
        A.parse_wav(make_wav(1, 1, 8000, 16, b"\0" * 8)[:24])


def test_float32_data_at_an_unaligned_offset():
    wav = make_wav(3, 1, 8000, 32, f32([1.0, -0.25, 0.5]), fmt_size=18, extra=(b"fact", struct.pack("<I", 3)))
    s, rate = A.parse_wav(wav)
    assert rate == 8000.0 and s.tolist() == [1.0, -0.25, 0.5]


def test_odd_chunks_are_word_aligned_and_headers_checked():
    wav = make_wav(3, 1, 8000, 32, f32([0.5]) * 11, extra=(b"LIST", b"abc\0\0"))  # 5-byte chunk + pad byte
    wav = wav.replace(b"abc\0\0data", b"abc\0\0\0data")
    wav = wav[:4] + struct.pack("<I", len(wav) - 8) + wav[8:]
    s, _ = A.parse_wav(wav)
    assert s.size == 11 and np.all(s == 0.5)
    with pytest.raises(A.AudioFileError, match="RIFF"):
        A.parse_wav(b"RIFX" + wav[4:])
    with pytest.raises(A.AudioFileError, match="too small"):
        A.parse_wav(wav[:40])
    for fmt, bits in ((1, 8), (3, 64), (2, 16)):
        with pytest.raises(A.AudioFileError, match="unsupported"):
            A.parse_wav(make_wav(fmt, 1, 8000, bits, b"\0" * 64))
    with pytest.raises(A.AudioFileError, match="file_not_found"):
        A.load("/nonexistent/x.wav")


def test_pcm_scaling_and_24_bit_sign_extension():
    s, _ = A.parse_wav(make_wav(1, 1, 8000, 16, struct.pack("<4h", -32768, 16384, 0, 32767)))
    assert s.tolist() == [-1.0, 0.5, 0.0, 32767 / 32768]
    raw = b"".join(v.to_bytes(3, "little") for v in (0x800000, 0x7FFFFF, 0xFFFFFF, 0x000001))
    s, _ = A.parse_wav(make_wav(1, 1, 8000, 24, raw))
    assert s.tolist() == [-1.0, 8388607 / 8388608, -1 / 8388608, 1 / 8388608]


def test_pcm16_matches_the_wave_module_and_mono_mixdown():
    rng = np.random.default_rng(0)
    pcm = rng.integers(-32768, 32768, (1000, 3), dtype=np.int16)
    buf = io.BytesIO()
    with wave.open(buf, "wb") as w:
        w.setnchannels(3)
        w.setsampwidth(2)
        w.setframerate(22050)
        w.writeframes(pcm.tobytes())
    s, rate = A.parse_wav(buf.getvalue(), mono=False)
    assert rate == 22050.0
    np.testing.assert_array_equal(s, (pcm.reshape(-1).astype(np.float32) / np.float32(32768)))
    m, _ = A.parse_wav(buf.getvalue(), mono=True)
    x = pcm.astype(np.float32) / np.float32(32768)
    ref = ((x[:, 0] + x[:, 1]) + x[:, 2]) * (np.float32(1) / np.float32(3))
    np.testing.assert_array_equal(m, ref.astype(np.float32))


def test_save_writes_the_reference_header_and_round_trips(tmp_path):
    x = np.random.default_rng(1).standard_normal(777).astype(np.float32)
    p = str(tmp_path / "a.wav")
    A.save(p, x, 44100.0)
    b = open(p, "rb").read()
    head = (b"RIFF" + struct.pack("<I", 36 + 4 * 777) + b"WAVE" + b"fmt " + struct.pack("<IHHIIHH", 16, 3, 1, 44100,
            44100 * 4, 4, 32) + b"data" + struct.pack("<I", 4 * 777))
    assert b[:44] == head and len(b) == 44 + 4 * 777
    s, rate = A.load(p)
    assert rate == 44100.0
    np.testing.assert_array_equal(s, x)


# ------------------------------------------------------------ checkpoints
def small_cfg():
    return HarmonicConfig(B=1, T=4096, K=8, NF=7, hidden=16, layers=2, din=3)


def test_snapshot_names_shapes_and_the_reference_initialisation():
    cfg = small_cfg()
    snaps = C.harmonic_snapshots(cfg, cfg.weights())
    assert [s.name for s in snaps] == ["W1", "b1", "W2", "b2", "W_harm", "b_harm", "W_gain", "b_gain", "W_noise",
                                       "b_noise", "W_noiseFilter", "b_noiseFilter"]
    assert [s.shape for s in snaps] == [[3, 16], [1, 16], [16, 16], [1, 16], [16, 8], [1, 8], [16, 1], [1, 1],
                                        [16, 1], [1, 1], [16, 7], [1, 7]]
    # HarmonicDecoderModel.init draws W1, W2, W_harm, W_gain, W_noise,
    # W_noiseFilter in that order from one SeededGenerator
    rng = SplitMix64(cfg.weight_seed)
    draws = [reference_random_array(rng, 3 * 16, np.float32(math.sqrt(2 / 3) * 0.5)),
             reference_random_array(rng, 16 * 16, np.float32(math.sqrt(2 / 16) * 0.5)),
             reference_random_array(rng, 16 * 8, 0.06), reference_random_array(rng, 16, 0.05),
             reference_random_array(rng, 16, 0.05), reference_random_array(rng, 16 * 7, 0.05)]
    for s, d in zip([snaps[i] for i in (0, 2, 4, 6, 8, 10)], draws):
        np.testing.assert_array_equal(s.data, d)
    assert snaps[9].data.tolist() == [-3.0]  # b_noise init


def test_checkpoint_round_trip_is_bit_exact(tmp_path):
    cfg = small_cfg()
    p = np.random.default_rng(2).standard_normal(cfg.param_count()).astype(np.float32)
    p[:5] = [0.0, 1e-30, -3.0, 1e20, 123456.789]
    path = C.write_model_state(str(tmp_path), 42, C.harmonic_snapshots(cfg, p), created_at="2026-01-02T03:04:05Z")
    assert os.path.basename(path) == "model_step_00000042.json"
    text = open(path).read()
    assert text.startswith('{\n  "createdAtUTC" : "2026-01-02T03:04:05Z",\n  "params" : [\n    {\n      "data" : [')
    assert '\n  "step" : 42\n}' in text
    ck = C.read_model_state(path)
    assert ck.step == 42 and ck.createdAtUTC == "2026-01-02T03:04:05Z"
    q = C.load_harmonic_snapshots(cfg, ck.params, np.zeros(cfg.param_count(), np.float32))
    np.testing.assert_array_equal(q, p)
    best = C.write_best_model_state(str(tmp_path), 7, ck.params)
    assert os.path.basename(best) == "model_best.json" and C.read_model_state(best).step == 7
    t = C.write_training_checkpoint(str(tmp_path), 3, 12, "a/b", created_at="x")
    assert os.path.basename(t) == "step_00000003.json"
    assert json.load(open(t)) == {"createdAtUTC": "x", "note": "a/b", "seenChunks": 12, "step": 3}
    assert '"a\\/b"' in open(t).read()  # JSONEncoder escapes '/'


def test_loading_skips_foreign_names_and_rejects_wrong_shapes(tmp_path):
    cfg = small_cfg()
    p = cfg.weights()
    snaps = C.harmonic_snapshots(cfg, p * 2)
    other = [C.NamedTensorSnapshot("tr_l0_wq", [2, 2], np.ones(4))] + [s for s in snaps if s.name == "W_harm"]
    q = C.load_harmonic_snapshots(cfg, other, p)
    assert np.array_equal(C.harmonic_snapshots(cfg, q)[4].data, snaps[4].data)
    assert np.array_equal(C.harmonic_snapshots(cfg, q)[0].data, C.harmonic_snapshots(cfg, p)[0].data)
    with pytest.raises(ValueError, match="shape"):
        C.load_harmonic_snapshots(cfg, [C.NamedTensorSnapshot("W_gain", [1, 16], np.zeros(16))], p)
    # a file in the reference's own spelling: integral floats, exponents
    path = tmp_path / "ref.json"
    path.write_text('{\n  "createdAtUTC" : "2026-05-01T00:00:00Z",\n  "params" : [\n    {\n      "data" : [\n'
                    '        0,\n        -3,\n        1e-07,\n        0.1\n      ],\n      "name" : "b_harm",\n'
                    '      "shape" : [\n        1,\n        4\n      ]\n    }\n  ],\n  "step" : 9\n}')
    ck = C.read_model_state(str(path))
    assert ck.params[0].data.tolist() == np.array([0, -3, 1e-7, 0.1], np.float32).tolist()


# -------------------------------------------------------------- dataset
def test_resample_normalize_and_window_starts():
    x = np.arange(10, dtype=np.float32)
    assert D.resample_linear(x, 24000.2, 24000.0) is not None and np.array_equal(D.resample_linear(x, 24000.2, 24000),
                                                                                 x)
    up = D.resample_linear(x, 12000.0, 24000.0)
    assert up.size == 20 and np.allclose(up[:19], np.arange(19) / 2) and up[19] == 9.0  # last clamps
    down = D.resample_linear(np.arange(9, dtype=np.float32), 48000, 16000)
    assert down.size == 3 and down.tolist() == [0.0, 3.0, 6.0]
    y = D.normalize_peak(np.array([0.1, -0.5, 0.25], np.float32), 0.99)
    assert abs(np.abs(y).max() - 0.99) < 1e-7 and D.normalize_peak(np.zeros(3, np.float32), 0.99).tolist() == [0] * 3
    assert D.start_indices(100, 200, 50) == [0]
    assert D.start_indices(1000, 256, 128) == [0, 128, 256, 384, 512, 640, 744]
    assert D.start_indices(512, 256, 128) == [0, 128, 256]


def test_features_of_silence_and_of_a_sine():
    cfg = D.make_config()
    sr = 24000.0
    f0, loud, uv = D.extract_features(np.zeros(4096, np.float32), sr, cfg)
    assert f0.size == 13 and np.all(f0 == 0) and np.all(uv == 0) and np.all(loud == -120.0)
    n = np.arange(8192)
    for hz, amp in ((220.0, 0.8), (331.7, 0.3), (612.0, 0.5)):
        x = (amp * np.sin(2 * np.pi * hz * n / sr)).astype(np.float32)
        f0, loud, uv = D.extract_features(x, sr, cfg)
        assert np.all(uv == 1)
        # the unnormalised autocorrelation's (n - lag) taper pulls the peak
        # ~1/((n - L0) w^2) lags short (220 Hz: +0.3% in f0), as in the reference
        assert np.abs(f0 / hz - 1).max() < 1e-2, (hz, f0)
        assert np.abs(loud - 20 * np.log10(amp / np.sqrt(2))).max() < 0.05
    # the autocorrelation is not normalised per lag, so a tone whose period
    # is long against the shortest lag (sr / maxF0 = 24) peaks there and is
    # reported unrefined as maxF0, as the reference's estimator does
    f0, _, uv = D.extract_features((0.3 * np.sin(2 * np.pi * 97.3 * n / sr)).astype(np.float32), sr, cfg)
    assert np.all(uv == 1) and np.all(f0 == np.float32(24000.0 / 24))


def test_f0_estimate_is_the_autocorrelation_peak():
    rng = np.random.default_rng(3)
    cfg = D.make_config()
    for _ in range(5):
        frame = (np.sin(2 * np.pi * rng.uniform(80, 900) * np.arange(1024) / 24000) +
                 0.3 * rng.standard_normal(1024)).astype(np.float32)
        c = frame.astype(np.float64) - frame.astype(np.float64).mean()
        lo, hi = int(24000 / 1000), min(1022, int(24000 / 50))
        corr = [np.dot(c[:1024 - L], c[L:]) for L in range(lo, hi + 1)]
        best = lo + int(np.argmax(corr))
        f, v = D.estimate_f0(frame, 24000.0, 50.0, 1000.0, 0.0005, 0.0)
        assert v and abs(24000.0 / f - best) <= 1.0  # the refined lag stays within one lag of the peak


def test_swift_shuffle_and_bounded_draws():
    rng = SplitMix64(1337)
    draws = [D.next_bounded(rng, b) for b in (1, 2, 3, 7, 1000, 2 ** 63 + 5) for _ in range(50)]
    bounds = [b for b in (1, 2, 3, 7, 1000, 2 ** 63 + 5) for _ in range(50)]
    assert all(0 <= d < b for d, b in zip(draws, bounds))
    # one draw per position: the first swap uses floor(x * n / 2^64) of the first draw
    first = SplitMix64(9).next()
    items = list(range(10))
    D.swift_shuffle(items, SplitMix64(9))
    assert sorted(items) == list(range(10)) and items[0] == (first * 10) >> 64
    a, b = list(range(50)), list(range(50))
    D.swift_shuffle(a, SplitMix64(5))
    D.swift_shuffle(b, SplitMix64(5))
    assert a == b and a != list(range(50))


def write_wavs(root):
    os.makedirs(os.path.join(root, "sub"), exist_ok=True)
    os.makedirs(os.path.join(root, ".hidden"), exist_ok=True)
    n = np.arange(30000)
    x = (0.4 * np.sin(2 * np.pi * 330 * n / 16000)).astype(np.float32)
    pcm = np.round(np.stack([x, x], 1) * 32767).astype(np.int16)
    with wave.open(os.path.join(root, "sub", "b.WAV"), "wb") as w:
        w.setnchannels(2)
        w.setsampwidth(2)
        w.setframerate(16000)
        w.writeframes(pcm.tobytes())
    A.save(os.path.join(root, "a.wav"), (0.2 * np.sin(2 * np.pi * 150 * np.arange(20000) / 24000)).astype(np.float32),
           24000.0)
    A.save(os.path.join(root, ".hidden", "c.wav"), np.zeros(100, np.float32), 24000.0)
    open(os.path.join(root, "notes.txt"), "w").write("x")


def test_cache_round_trip_and_training_batch(tmp_path):
    root, cache = str(tmp_path / "in"), str(tmp_path / "cache")
    write_wavs(root)
    files = D.find_wav_files(root)
    assert [os.path.relpath(f, root) for f in files] == ["a.wav", "sub/b.WAV"]
    m = D.preprocess(root, cache, {"chunkSize": 16384, "chunkHop": 8192}, created_at="t")
    # a.wav: 20000 samples -> starts 0, 3616; b.WAV: 30000 at 16 kHz -> 45000 -> 0, 8192, 16384, 24576, 28616
    assert m["chunkCount"] == 7 and m["trainCount"] + m["valCount"] == 7 and m["valCount"] == 1
    text = open(os.path.join(cache, "manifest.json")).read()
    # JSONEncoder with .sortedKeys: compact, keys in order
    assert text.startswith('{"chunkCount":7,"config":{') and '": ' not in text and '", "' not in text
    ds = D.CachedDataset.load(cache)
    assert len(ds.entries()) == 7 and len(ds.entries("train")) == 6 and len(ds.entries("val")) == 1
    assert "maxFiles" not in ds.manifest["config"] and ds.manifest["config"]["seed"] == 1337
    e = [x for x in ds.entries() if x["sourceFile"] == os.path.join("sub", "b.WAV")]
    assert [x["startSample"] for x in e] == [0, 8192, 16384, 24576, 28616]
    assert all(x["sourceSampleRate"] == 16000.0 and x["featureFrames"] == 61 for x in e)
    c = ds.load_chunk(e[0])
    assert c["audio"].size == 16384 and abs(np.abs(c["audio"]).max() - 0.99) < 1e-6
    voiced = c["uvMask"] > 0
    assert voiced.all() and np.abs(c["f0Hz"] / 330 - 1).max() < 1e-2
    cfg = D.make_config()
    f0, uv, X, tgt = D.harmonic_batch([c, ds.load_chunk(e[-1])], cfg, 64, 16384)
    assert f0.shape == (64, 2) and X.shape == (128, 3) and tgt.shape == (2, 16384)
    assert np.all(f0[61:, 0] == c["f0Hz"][60]) and np.all(X[61:64] == 0)  # padded frames
    fn = (np.log(np.float32(c["f0Hz"][3])) - np.log(np.float32(50))) / (np.log(np.float32(1000)) -
                                                                          np.log(np.float32(50)))
    assert abs(X[3, 0] - fn) < 1e-6 and abs(X[3, 1] - min(max((c["loudnessDB"][3] + 80) / 80, 0), 1)) < 1e-7
    assert X[3, 2] == 1.0 and np.array_equal(tgt[0], c["audio"])
