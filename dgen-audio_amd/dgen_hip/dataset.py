"""The HarmonicE2E dataset cache: preprocessing of a folder of WAV files into
``manifest.json`` + ``chunks/chunk_%08d.json``, its reader, and the batch
assembly that feeds cached chunks to a training step.

Follows Examples/HarmonicE2E/Dataset.swift (DatasetPreprocessor.preprocess
:56-165: find .wav files, load mono, linear resample to the config rate,
peak-normalise, cut chunkSize chunks every chunkHop samples (a last chunk
aligned to the end, zero padding for short files), extract features,
assign train/val splits), Features.swift (FeatureExtractor: per-frame RMS
loudness in dB and an autocorrelation f0 estimate with parabolic lag
refinement) and Trainer.swift (makeConditioningData :589-617 and the
batched f0 / uv / audio interleave :320-353).  Every Float computation keeps
the reference's fp32 operation order (sums run sequentially).

The manifest and chunk files are written as JSONEncoder writes them with
``.sortedKeys`` (compact), so the reference's ``CachedDataset`` can read a
cache written here and this reader reads one written there.

Chunk shuffling (``shuffleChunks``) restates the Swift standard library's
published ``shuffle(using:)`` (forward Fisher-Yates) with Lemire's bounded
draw (``next(upperBound:)``) over the HarmonicE2E SeededGenerator
(SplitMix64, Config.swift:244-260).  With no Swift toolchain here, that
order is checked against the algorithm's properties, not against Swift.
"""
from __future__ import annotations

import math
import os

import numpy as np

from . import audiofile
from .checkpoint import encode
from .workloads import SplitMix64

_M64 = (1 << 64) - 1

# HarmonicE2EConfig (Examples/HarmonicE2E/Config.swift:3-39) with its defaults;
# maxFiles / maxChunksPerFile are optional (absent = no limit).
DEFAULT_CONFIG = {
    "sampleRate": 24000.0, "chunkSize": 16384, "chunkHop": 8192, "frameSize": 1024, "frameHop": 256,
    "minF0Hz": 50.0, "maxF0Hz": 1000.0, "silenceRMS": 0.0005, "voicedThreshold": 0.3, "peakNormalizeTo": 0.99,
    "trainSplit": 0.9, "shuffleChunks": True, "seed": 1337, "maxFiles": None, "maxChunksPerFile": None,
    "modelHiddenSize": 64, "modelNumLayers": 2, "numHarmonics": 32, "noiseFilterSize": 63, "batchSize": 1,
    "harmonicPathScale": 1.0, "noisePathScale": 1.0, "learningRate": 0.001, "mseLossWeight": 0.0,
    "spectralWeight": 1.0, "spectralLogmagWeight": 0.5, "spectralWindowSizes": [128, 256, 512],
    "spectralHopDivisor": 4, "logEvery": 10, "checkpointEvery": 100,
}
FLOAT_KEYS = {"sampleRate", "minF0Hz", "maxF0Hz", "silenceRMS", "voicedThreshold", "peakNormalizeTo", "trainSplit",
              "harmonicPathScale", "noisePathScale", "learningRate", "mseLossWeight", "spectralWeight",
              "spectralLogmagWeight"}


def make_config(**overrides) -> dict:
    """A HarmonicE2EConfig: the defaults, then ``overrides`` (decoding a
    config keeps the default of every absent key, Config.swift:76-128)."""
    cfg = dict(DEFAULT_CONFIG)
    for k, v in overrides.items():
        if k not in cfg:
            raise KeyError(f"unknown HarmonicE2EConfig key {k}")
        cfg[k] = v
    return cfg


def _f32(v) -> np.float32:
    return np.float32(v)


# -------------------------------------------------- Swift random shuffles
def next_bounded(rng: SplitMix64, bound: int) -> int:
    """RandomNumberGenerator.next(upperBound:): Lemire's nearly divisionless
    method on the 64-bit draw (high word of draw * bound, rejecting low words
    below (2^64 - bound) mod bound)."""
    if bound <= 0:
        raise ValueError("upper bound must be positive")
    m = rng.next() * bound
    if (m & _M64) < bound:
        t = ((1 << 64) - bound) % bound
        while (m & _M64) < t:
            m = rng.next() * bound
    return m >> 64


def swift_shuffle(items: list, rng: SplitMix64) -> None:
    """MutableCollection.shuffle(using:) in place: for each position from the
    front, swap it with a uniformly drawn position among those not yet fixed."""
    amount, cur = len(items), 0
    while amount > 1:
        r = next_bounded(rng, amount)
        amount -= 1
        items[cur], items[cur + r] = items[cur + r], items[cur]
        cur += 1


# --------------------------------------------------- signal preprocessing
def resample_linear(samples: np.ndarray, source_rate: float, target_rate: float) -> np.ndarray:
    """Dataset.swift resampleLinear (:255-273), in fp32."""
    x = np.ascontiguousarray(samples, np.float32)
    if x.size == 0:
        return x
    sr, tr = _f32(source_rate), _f32(target_rate)
    if abs(float(sr) - float(tr)) < 0.5:
        return x
    ratio = _f32(tr / sr)
    prod = float(_f32(_f32(x.size) * ratio))
    count = max(1, int(math.floor(abs(prod) + 0.5)) * (1 if prod >= 0 else -1))  # .rounded(): half away from 0
    pos = (np.arange(count, dtype=np.float32) / ratio).astype(np.float32)
    i0 = np.floor(pos).astype(np.int64)
    i1 = np.minimum(i0 + 1, x.size - 1)
    frac = (pos - i0.astype(np.float32)).astype(np.float32)
    a = x[np.clip(i0, 0, x.size - 1)]
    b = x[i1]
    return (a + ((b - a).astype(np.float32) * frac).astype(np.float32)).astype(np.float32)


def normalize_peak(samples: np.ndarray, peak_target: float) -> np.ndarray:
    """Dataset.swift normalizePeak (:275-281)."""
    x = np.ascontiguousarray(samples, np.float32)
    if x.size == 0:
        return x
    peak = np.abs(x).max()
    if not peak > 0:
        return x
    return (x * _f32(_f32(peak_target) / peak)).astype(np.float32)


def start_indices(count: int, size: int, hop: int) -> list:
    """Window starts every ``hop`` while a whole window fits, plus one window
    ending at the last sample (Dataset.swift chunkStartIndices :201-214;
    Features.swift makeFrameStarts :48-62, which returns [0] for an empty
    signal where the chunker returns none)."""
    if count <= size:
        return [0]
    starts = list(range(0, count - size + 1, hop))
    if starts and starts[-1] + size < count:
        starts.append(max(0, count - size))
    return starts


def _seq_sum(v: np.ndarray) -> np.float32:
    """A sequential fp32 sum (the reference's `for x in ... { sum += x }`)."""
    return np.cumsum(np.asarray(v, np.float32), dtype=np.float32)[-1] if v.size else np.float32(0.0)


def rms(frame: np.ndarray) -> np.float32:
    f = np.asarray(frame, np.float32)
    if f.size == 0:
        return np.float32(0.0)
    return np.sqrt(_seq_sum((f * f).astype(np.float32)) / _f32(f.size)).astype(np.float32)


def estimate_f0(frame: np.ndarray, sample_rate: float, min_f0: float, max_f0: float, silence_rms: float,
                voiced_threshold: float) -> tuple[float, bool]:
    """Features.swift estimateF0Autocorr (:84-153): normalised autocorrelation
    of the mean-removed frame over lags [sr/maxF0, sr/minF0], the best lag
    refined by a parabola through its neighbours."""
    f = np.asarray(frame, np.float32)
    if rms(f) < _f32(silence_rms):
        return 0.0, False
    mean = _f32(_seq_sum(f) / _f32(f.size))
    c = (f - mean).astype(np.float32)
    energy = _seq_sum((c * c).astype(np.float32))
    if energy <= _f32(1e-8):
        return 0.0, False
    sr = _f32(sample_rate)
    min_lag = max(1, int(float(_f32(sr / _f32(max_f0)))))
    max_lag = min(c.size - 2, int(float(_f32(sr / _f32(min_f0)))))
    if max_lag <= min_lag:
        return 0.0, False
    n = c.size
    lags = np.arange(min_lag, max_lag + 1)
    # products c[i] c[i + lag] for i < n - lag, zero beyond; sequential sums per lag
    idx = np.arange(n)[None, :] + lags[:, None]
    prod = np.where(idx < n, c[None, :] * c[np.minimum(idx, n - 1)], np.float32(0.0)).astype(np.float32)
    sums = np.cumsum(prod, axis=1, dtype=np.float32)[:, -1]
    corr = np.zeros(max_lag + 1, np.float32)
    corr[min_lag:] = (sums / _f32(energy + _f32(1e-8))).astype(np.float32)
    best = min_lag + int(np.argmax(corr[min_lag:]))  # the first of equal maxima (strict >)
    if corr[best] < _f32(voiced_threshold):
        return 0.0, False
    lag = _f32(best)
    if min_lag < best < max_lag:
        y0, y1, y2 = corr[best - 1], corr[best], corr[best + 1]
        denom = _f32(_f32(y0 - _f32(2.0 * y1)) + y2)
        if abs(float(denom)) > 1e-8:
            delta = _f32(_f32(0.5) * _f32(y0 - y2) / denom)
            lag = _f32(lag + _f32(max(-1.0, min(1.0, float(delta)))))
    return float(_f32(sr / _f32(max(float(lag), 1.0)))), True


def extract_features(samples: np.ndarray, sample_rate: float, cfg: dict):
    """FeatureExtractor.extract: per frame (frameSize every frameHop, zero
    padded) the loudness max(-120, 20 log10(max(rms, 1e-7))) in dB, f0 and
    the voiced flag.  Returns (f0Hz, loudnessDB, uvMask) float32."""
    x = np.asarray(samples, np.float32)
    size, hop = int(cfg["frameSize"]), int(cfg["frameHop"])
    f0, loud, uv = [], [], []
    for s in start_indices(x.size, size, hop):
        frame = np.zeros(size, np.float32)
        seg = x[s:s + size]
        frame[:seg.size] = seg
        r = rms(frame)
        loud.append(max(np.float32(-120.0), _f32(20.0 * np.log10(max(r, np.float32(1e-7)), dtype=np.float32))))
        p, v = estimate_f0(frame, sample_rate, cfg["minF0Hz"], cfg["maxF0Hz"], cfg["silenceRMS"],
                           cfg["voicedThreshold"])
        f0.append(p)
        uv.append(1.0 if v else 0.0)
    return np.array(f0, np.float32), np.array(loud, np.float32), np.array(uv, np.float32)


# ------------------------------------------------------------ the cache
def find_wav_files(root: str, max_files=None, shuffle: bool = False, seed: int = 0) -> list:
    """Every *.wav (any case) under root, hidden files and folders skipped,
    sorted by path, then shuffled with the seed and cut to max_files."""
    files = []
    for d, dirs, names in os.walk(root):
        dirs[:] = [x for x in dirs if not x.startswith(".")]
        files += [os.path.join(d, n) for n in names if not n.startswith(".") and n.lower().endswith(".wav")]
    files.sort()
    if shuffle:
        swift_shuffle(files, SplitMix64(seed))
    if max_files is not None and len(files) > max_files:
        files = files[:max_files]
    return files


def assign_splits(entries: list, train_split: float, seed: int, shuffle: bool) -> None:
    """Dataset.swift assignSplits (:216-235): the first floor(n * trainSplit)
    positions of the (shuffled) order are train, at least one of each when
    there are two or more chunks."""
    if not entries:
        return
    order = list(range(len(entries)))
    if shuffle:
        swift_shuffle(order, SplitMix64(seed))
    n_train = int(math.floor(float(_f32(_f32(len(entries)) * _f32(train_split)))))
    n_train = max(1, min(len(entries) - 1, n_train))
    if len(entries) == 1:
        n_train = 1
    for pos, i in enumerate(order):
        entries[i]["split"] = "train" if pos < n_train else "val"


def _write_json(path: str, value) -> None:
    tmp = path + ".tmp"
    with open(tmp, "w", encoding="utf-8") as fh:
        fh.write(encode(value, pretty=False))
    os.replace(tmp, path)


def _config_json(cfg: dict) -> dict:
    out = {}
    for k, v in cfg.items():
        if v is None:
            continue  # optionals are omitted when nil
        out[k] = float(_f32(v)) if k in FLOAT_KEYS else v
    return out


def preprocess(input_root: str, cache_root: str, cfg: dict | None = None, logger=None,
               created_at: str | None = None) -> dict:
    """DatasetPreprocessor.preprocess: writes the chunk files and the
    manifest under cache_root and returns the manifest."""
    from .checkpoint import utc_now
    cfg = make_config(**(cfg or {}))
    log = logger or (lambda s: None)
    files = find_wav_files(input_root, cfg["maxFiles"], cfg["shuffleChunks"], cfg["seed"])
    if not files:
        raise ValueError(f"No .wav files found in {input_root}")
    chunks_dir = os.path.join(cache_root, "chunks")
    os.makedirs(chunks_dir, exist_ok=True)
    log(f"Found {len(files)} wav files")
    rate = float(_f32(cfg["sampleRate"]))
    size, hop = int(cfg["chunkSize"]), int(cfg["chunkHop"])
    entries, index = [], 0
    root_abs = os.path.abspath(input_root)
    for fi, path in enumerate(files):
        rel = os.path.relpath(os.path.abspath(path), root_abs)
        log(f"[{fi + 1}/{len(files)}] {rel}")
        raw, src_rate = audiofile.load(path, mono=True)
        x = normalize_peak(resample_linear(raw, src_rate, rate), cfg["peakNormalizeTo"])
        written = 0
        for start in (start_indices(x.size, size, hop) if x.size else []):
            if cfg["maxChunksPerFile"] is not None and written >= cfg["maxChunksPerFile"]:
                break
            chunk = np.zeros(size, np.float32)
            seg = x[start:start + size]
            chunk[:seg.size] = seg
            f0, loud, uv = extract_features(chunk, rate, cfg)
            cid = "chunk_%08d" % index
            record = {"id": cid, "sourceFile": rel, "sourceSampleRate": src_rate, "sampleRate": rate,
                      "startSample": int(start), "audio": chunk, "f0Hz": f0, "loudnessDB": loud, "uvMask": uv}
            _write_json(os.path.join(chunks_dir, cid + ".json"), record)
            entries.append({"id": cid, "split": "train", "sourceFile": rel, "sourceSampleRate": src_rate,
                            "startSample": int(start), "chunkSamples": int(chunk.size),
                            "featureFrames": int(f0.size), "relativeChunkPath": f"chunks/{cid}.json"})
            index += 1
            written += 1
    if not entries:
        raise ValueError("No chunks were generated. Check chunk size/hop and audio length")
    assign_splits(entries, cfg["trainSplit"], cfg["seed"], cfg["shuffleChunks"])
    n_train = sum(e["split"] == "train" for e in entries)
    manifest = {"version": 1, "createdAtUTC": created_at or utc_now(), "sourceRoot": root_abs,
                "config": _config_json(cfg), "chunkCount": len(entries), "trainCount": n_train,
                "valCount": len(entries) - n_train, "entries": entries}
    _write_json(os.path.join(cache_root, "manifest.json"), manifest)
    log(f"Chunks: total={len(entries)} train={n_train} val={len(entries) - n_train}")
    return manifest


class CachedDataset:
    """A written cache (Dataset.swift CachedDataset :287-308)."""

    def __init__(self, root: str, manifest: dict):
        self.root, self.manifest = root, manifest

    @classmethod
    def load(cls, root: str) -> "CachedDataset":
        import json
        with open(os.path.join(root, "manifest.json"), "r", encoding="utf-8") as fh:
            return cls(root, json.load(fh))

    def entries(self, split: str | None = None) -> list:
        e = self.manifest["entries"]
        return list(e) if split is None else [x for x in e if x["split"] == split]

    def load_chunk(self, entry: dict) -> dict:
        import json
        with open(os.path.join(self.root, entry["relativeChunkPath"]), "r", encoding="utf-8") as fh:
            c = json.load(fh)
        for k in ("audio", "f0Hz", "loudnessDB", "uvMask"):
            c[k] = np.array(c[k], np.float64).astype(np.float32)
        return c


# ------------------------------------------------------ training batches
def conditioning(chunk: dict, cfg: dict, frames: int) -> np.ndarray:
    """Trainer.swift makeConditioningData (:589-617): per frame [f0 norm,
    loudness norm, uv] with f0 norm = (log max(f0, minF0) - log max(minF0, 1))
    / span on voiced frames (0 else), loudness (dB + 80) / 80 clipped to
    [0, 1]; frames past the chunk's are zero.  [frames][3] float32."""
    min_log = math.log(max(float(_f32(cfg["minF0Hz"])), 1.0))
    max_log = math.log(max(float(_f32(cfg["maxF0Hz"])), float(_f32(cfg["minF0Hz"])) + 1.0))
    min_log, max_log = float(_f32(min_log)), float(_f32(max_log))
    span = _f32(max(1e-6, float(_f32(max_log - min_log))))
    out = np.zeros((frames, 3), np.float32)
    f0, loud, uv = chunk["f0Hz"], chunk["loudnessDB"], chunk["uvMask"]
    for i in range(min(frames, f0.size)):
        f = max(f0[i], _f32(cfg["minF0Hz"]))
        fn = _f32(_f32(_f32(math.log(float(f))) - _f32(min_log)) / span) if uv[i] > 0.5 else np.float32(0.0)
        ln = min(max(_f32(_f32(loud[i] + _f32(80.0)) / _f32(80.0)), np.float32(0.0)), np.float32(1.0))
        out[i] = (fn, ln, uv[i])
    return out


def harmonic_batch(chunks: list, cfg: dict, frames: int, frame_count: int):
    """One training batch from B cached chunks (Trainer.swift :320-353):
    returns (f0 [F][B], uv [F][B], X [B*F][3] with row b*F + f, target
    [B][frame_count]); a chunk's f0 and uv repeat its last frame past its
    end, its audio is zero past its end."""
    B = len(chunks)
    f0 = np.zeros((frames, B), np.float32)
    uv = np.zeros((frames, B), np.float32)
    X = np.zeros((B * frames, 3), np.float32)
    target = np.zeros((B, frame_count), np.float32)
    for b, c in enumerate(chunks):
        X[b * frames:(b + 1) * frames] = conditioning(c, cfg, frames)
        n = c["f0Hz"].size
        if n:
            src = np.minimum(np.arange(frames), n - 1)
            f0[:, b] = c["f0Hz"][src]
            uv[:, b] = c["uvMask"][src]
        a = c["audio"][:frame_count]
        target[b, :a.size] = a
    return f0, uv, X, target
