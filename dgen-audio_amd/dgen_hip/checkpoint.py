"""Model checkpoints in the reference's JSON format.

``ModelCheckpoint {step, createdAtUTC, params: [NamedTensorSnapshot]}`` and
``NamedTensorSnapshot {name, shape, data}`` (Examples/HarmonicE2E/Model.swift:
11-15, Checkpoint.swift:3-43; Examples/DDSPE2E/Checkpoint.swift:1-83 adds
``TrainingCheckpoint {step, createdAtUTC, note, seenChunks}``), written like
Swift's JSONEncoder with ``[.prettyPrinted, .sortedKeys]`` ("key" : value,
two-space indent, sorted keys) to ``model_step_%08d.json`` /
``model_best.json`` / ``step_%08d.json``.  Floats are written as the
shortest decimal that reads back as the same float32 (integral values
without a fraction, as Swift writes them), so a checkpoint round-trips bit
for bit.

The HarmonicE2E decoder's snapshots (HarmonicDecoderModel.snapshots,
Model.swift:122-141) name the tensors W1, b1, ... WL, bL, W_harm, b_harm,
W_gain, b_gain, W_noise, b_noise, W_noiseFilter, b_noiseFilter with shapes
[fanIn, hidden], [1, hidden], [hidden, K], [1, K], [hidden, 1], [1, 1],
[hidden, 1], [1, 1], [hidden, NF], [1, NF].  This build keeps the same
parameters as one blob (W1 b1 ... WL bL Wh bh, the four heads side by side
in Wh's columns), so ``harmonic_snapshots`` and ``load_harmonic_snapshots``
translate between the two.
"""
from __future__ import annotations

import datetime
import json
import math
import os
from dataclasses import dataclass, field

import numpy as np

from .workloads import HarmonicConfig


@dataclass
class NamedTensorSnapshot:
    name: str
    shape: list
    data: np.ndarray  # float32, flat

    def __post_init__(self):
        self.shape = [int(s) for s in self.shape]
        self.data = np.ascontiguousarray(self.data, np.float32).reshape(-1)
        if int(np.prod(self.shape)) != self.data.size:
            raise ValueError(f"snapshot {self.name}: shape {self.shape} does not hold {self.data.size} values")


@dataclass
class ModelCheckpoint:
    step: int
    params: list = field(default_factory=list)  # [NamedTensorSnapshot]
    createdAtUTC: str = ""


def utc_now() -> str:
    """ISO 8601 in UTC to the second, as ISO8601DateFormatter writes it."""
    return datetime.datetime.now(datetime.timezone.utc).strftime("%Y-%m-%dT%H:%M:%SZ")


# ------------------------------------------------------------- JSON writer
def _float(v) -> str:
    f = np.float32(v)
    if not math.isfinite(float(f)):
        raise ValueError("non-finite value in a checkpoint (JSONEncoder rejects it)")
    if float(f) == int(float(f)) and abs(float(f)) < 2.0 ** 63:
        return str(int(float(f)))
    s = np.format_float_scientific(f, unique=True, trim="-") if abs(float(f)) < 1e-4 or abs(float(f)) >= 1e16 \
        else np.format_float_positional(f, unique=True, trim="-")
    return s


def _dump(v, indent: int, pretty: bool) -> str:
    pad, step = ("\n" + " " * indent, " " * 2) if pretty else ("", "")
    sep, colon = ("," , " : ") if pretty else (",", ":")
    if isinstance(v, dict):
        if not v:
            return "{}"
        keys = sorted(v)
        inner = [f"{pad}{step}{json.dumps(k)}{colon}{_dump(v[k], indent + 2, pretty)}" for k in keys]
        return "{" + sep.join(inner) + pad + "}"
    if isinstance(v, (list, tuple, np.ndarray)):
        items = list(v)
        if not items:
            return "[]"
        inner = [f"{pad}{step}{_dump(x, indent + 2, pretty)}" for x in items]
        return "[" + sep.join(inner) + pad + "]"
    if isinstance(v, (bool, np.bool_)):
        return "true" if v else "false"
    if isinstance(v, (int, np.integer)):
        return str(int(v))
    if isinstance(v, (float, np.floating)):
        return _float(v)
    if isinstance(v, str):
        return json.dumps(v).replace("/", "\\/")  # JSONEncoder escapes '/'
    if v is None:
        return "null"
    raise TypeError(f"cannot encode {type(v)}")


def encode(value, pretty: bool = True) -> str:
    """JSON text as JSONEncoder writes it with .sortedKeys (and
    .prettyPrinted when ``pretty``)."""
    return _dump(value, 0, pretty)


def _write_atomic(path: str, text: str) -> None:
    tmp = path + ".tmp"
    with open(tmp, "w", encoding="utf-8") as fh:
        fh.write(text)
    os.replace(tmp, path)


def _snap_dict(s: NamedTensorSnapshot) -> dict:
    return {"name": s.name, "shape": list(s.shape), "data": [float(x) for x in s.data]}


# -------------------------------------------------------- store (files)
def write_model_state(checkpoints_dir: str, step: int, params, created_at: str | None = None) -> str:
    """model_step_%08d.json (CheckpointStore.writeModelState)."""
    ck = {"step": int(step), "createdAtUTC": created_at or utc_now(), "params": [_snap_dict(s) for s in params]}
    path = os.path.join(checkpoints_dir, "model_step_%08d.json" % step)
    _write_atomic(path, encode(ck))
    return path


def write_best_model_state(checkpoints_dir: str, step: int, params, created_at: str | None = None) -> str:
    """model_best.json (CheckpointStore.writeBestModelState)."""
    ck = {"step": int(step), "createdAtUTC": created_at or utc_now(), "params": [_snap_dict(s) for s in params]}
    path = os.path.join(checkpoints_dir, "model_best.json")
    _write_atomic(path, encode(ck))
    return path


def write_training_checkpoint(checkpoints_dir: str, step: int, seen_chunks: int, note: str,
                              created_at: str | None = None) -> str:
    """step_%08d.json (DDSPE2E CheckpointStore.writePlaceholder)."""
    ck = {"step": int(step), "createdAtUTC": created_at or utc_now(), "note": note, "seenChunks": int(seen_chunks)}
    path = os.path.join(checkpoints_dir, "step_%08d.json" % step)
    _write_atomic(path, encode(ck))
    return path


def read_model_state(path: str) -> ModelCheckpoint:
    """CheckpointStore.readModelState: every key required, data as float32."""
    with open(path, "r", encoding="utf-8") as fh:
        raw = json.load(fh)
    for key in ("step", "createdAtUTC", "params"):
        if key not in raw:
            raise ValueError(f"{path}: checkpoint has no '{key}'")
    params = []
    for p in raw["params"]:
        for key in ("name", "shape", "data"):
            if key not in p:
                raise ValueError(f"{path}: snapshot has no '{key}'")
        params.append(NamedTensorSnapshot(p["name"], p["shape"], np.array(p["data"], np.float64).astype(np.float32)))
    return ModelCheckpoint(int(raw["step"]), params, str(raw["createdAtUTC"]))


# ------------------------------------------------ HarmonicE2E parameters
def _layout(cfg: HarmonicConfig):
    """(name, shape, blob offset, column slice of Wh or None) per snapshot."""
    out, off, fan, H = [], 0, cfg.din, cfg.hidden
    for i in range(cfg.layers):
        out.append((f"W{i + 1}", [fan, H], off, None))
        off += fan * H
        out.append((f"b{i + 1}", [1, H], off, None))
        off += H
        fan = H
    wh, bh = off, off + H * cfg.NC
    K, NF = cfg.K, cfg.NF
    heads = [("harm", 0, K), ("gain", K, K + 1), ("noise", K + 1, K + 2), ("noiseFilter", K + 2, K + 2 + NF)]
    for name, c0, c1 in heads:
        out.append((f"W_{name}", [H, c1 - c0], wh, (c0, c1)))
        out.append((f"b_{name}", [1, c1 - c0], bh, (c0, c1)))
    return out


def harmonic_snapshots(cfg: HarmonicConfig, params) -> list:
    """The decoder's snapshots (HarmonicDecoderModel.snapshots order) from a
    parameter blob."""
    p = np.ascontiguousarray(params, np.float32).reshape(-1)
    if p.size != cfg.param_count():
        raise ValueError(f"parameter blob has {p.size} values, the model {cfg.param_count()}")
    H, NC = cfg.hidden, cfg.NC
    snaps = []
    for name, shape, off, cols in _layout(cfg):
        if cols is None:
            data = p[off:off + int(np.prod(shape))]
        elif name.startswith("W_"):
            data = p[off:off + H * NC].reshape(H, NC)[:, cols[0]:cols[1]]
        else:
            data = p[off:off + NC][cols[0]:cols[1]]
        snaps.append(NamedTensorSnapshot(name, shape, np.array(data)))
    return snaps


def load_harmonic_snapshots(cfg: HarmonicConfig, snapshots, params) -> np.ndarray:
    """A new blob: ``params`` with every tensor that ``snapshots`` names
    replaced.  Names the model does not have are skipped (as a decoder
    loading another backbone's snapshots skips them); a known name with
    another shape is an error."""
    p = np.array(params, np.float32).reshape(-1)
    if p.size != cfg.param_count():
        raise ValueError(f"parameter blob has {p.size} values, the model {cfg.param_count()}")
    H, NC = cfg.hidden, cfg.NC
    by_name = {name: (shape, off, cols) for name, shape, off, cols in _layout(cfg)}
    for s in snapshots:
        if s.name not in by_name:
            continue
        shape, off, cols = by_name[s.name]
        if list(s.shape) != shape:
            raise ValueError(f"snapshot {s.name}: shape {s.shape}, the model's is {shape}")
        if cols is None:
            p[off:off + s.data.size] = s.data
        elif s.name.startswith("W_"):
            p[off:off + H * NC].reshape(H, NC)[:, cols[0]:cols[1]] = s.data.reshape(shape)
        else:
            p[off:off + NC][cols[0]:cols[1]] = s.data
    return p
