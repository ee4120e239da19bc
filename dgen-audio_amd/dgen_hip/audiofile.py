"""WAV file I/O, the host side of DGenLazy's AudioFile
(Sources/DGenLazy/AudioFile.swift:34-233).

``load`` / ``parse_wav`` read RIFF/WAVE files: PCM int16 and int24 and IEEE
float32, any channel count, optionally mixed down to mono.  Like the
reference parser they walk the chunk list (word-aligned), take the first
"fmt " and "data" chunks, never trust the declared data size (it is clamped
to the bytes present, as streaming encoders write 0 or 0xFFFFFFFF there),
floor the payload to whole frames and read every value unaligned.  ``save``
writes the reference's 44-byte header and 32-bit float mono samples.
Malformed files raise ``AudioFileError``, never an out-of-range read.
"""
from __future__ import annotations

import os
import struct
import tempfile

import numpy as np


class AudioFileError(Exception):
    """Invalid, missing or unsupported WAV input (AudioFile.AudioFileError)."""

    def __init__(self, kind: str, message: str):
        super().__init__(f"{kind}: {message}")
        self.kind = kind  # "invalid_format", "file_not_found" or "unsupported_format"


def load(path: str, mono: bool = True) -> tuple[np.ndarray, float]:
    """(samples float32, sample rate).  Multi-channel files come back
    interleaved [frames * channels] unless ``mono``."""
    if not os.path.isfile(path):
        raise AudioFileError("file_not_found", path)
    with open(path, "rb") as fh:
        return parse_wav(fh.read(), mono)


def parse_wav(data: bytes, mono: bool = True) -> tuple[np.ndarray, float]:
    """Parse WAV bytes (AudioFile.parseWAV, AudioFile.swift:109-233)."""
    data = bytes(data)
    if len(data) < 44:
        raise AudioFileError("invalid_format", "File too small for WAV header")
    if data[0:4] != b"RIFF" or data[8:12] != b"WAVE":
        raise AudioFileError("invalid_format", "Missing RIFF/WAVE header")
    fmt = None
    data_off = data_size = None
    off = 12
    while off + 8 <= len(data):
        cid = data[off:off + 4]
        size = struct.unpack_from("<I", data, off + 4)[0]
        start = off + 8
        if cid == b"fmt ":
            if size < 16 or start + 16 > len(data):
                raise AudioFileError("invalid_format", "fmt chunk truncated")
            fmt = struct.unpack_from("<HHIIHH", data, start)  # format, channels, rate, byte rate, align, bits
        elif cid == b"data":
            data_off, data_size = start, size
        off = start + size + (size & 1)  # chunks are word-aligned
        if fmt is not None and data_off is not None:
            break
    if fmt is None:
        raise AudioFileError("invalid_format", "No fmt chunk found")
    if data_off is None:
        raise AudioFileError("invalid_format", "No data chunk found")
    audio_format, channels, rate, _, _, bits = fmt
    if channels < 1:
        raise AudioFileError("invalid_format", "Invalid channel count")
    if data_off >= len(data):
        raise AudioFileError("invalid_format", "data chunk offset past end of file")
    data_size = min(data_size, len(data) - data_off)

    def whole_frames(bytes_per_sample: int) -> int:
        frame = channels * bytes_per_sample
        usable = (data_size // frame) * frame
        if usable <= 0:
            raise AudioFileError("invalid_format", "data chunk has no complete frames")
        return usable // bytes_per_sample

    if audio_format == 1:
        if bits not in (16, 24):
            raise AudioFileError("unsupported_format", f"PCM {bits}-bit (only 16-bit and 24-bit supported)")
        bps = bits // 8
        n = whole_frames(bps)
        raw = np.frombuffer(data, np.uint8, n * bps, data_off)
        if bits == 16:
            v = raw.view("<i2").astype(np.float32)
            samples = (v / np.float32(32768.0)).astype(np.float32)
        else:
            b = raw.reshape(n, 3).astype(np.int32)
            v = b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16)
            v = np.where(v & 0x800000, v | ~0xFFFFFF, v)  # sign-extend 24 bits
            samples = (v.astype(np.float32) / np.float32(8388608.0)).astype(np.float32)
    elif audio_format == 3:
        if bits != 32:
            raise AudioFileError("unsupported_format", f"Float {bits}-bit (only 32-bit supported)")
        n = whole_frames(4)
        samples = np.frombuffer(data, "<f4", n, data_off).astype(np.float32)
    else:
        raise AudioFileError("unsupported_format",
                             f"audioFormat {audio_format} (only PCM int16 and float32 supported)")
    if mono and channels > 1:
        frames = samples.reshape(-1, channels)
        acc = np.zeros(frames.shape[0], np.float32)
        for ch in range(channels):  # the reference's channel order, fp32
            acc = (acc + frames[:, ch]).astype(np.float32)
        samples = (acc * (np.float32(1.0) / np.float32(channels))).astype(np.float32)
    return samples, float(np.float32(rate))


def wav_bytes(samples, sample_rate: float) -> bytes:
    """The bytes ``save`` writes: RIFF header, fmt (IEEE float, mono,
    32-bit), data (AudioFile.save, AudioFile.swift:58-104)."""
    s = np.ascontiguousarray(samples, np.float32).reshape(-1)
    rate = int(np.float32(sample_rate))
    n = s.size * 4
    head = b"RIFF" + struct.pack("<I", 36 + n) + b"WAVE"
    head += b"fmt " + struct.pack("<IHHIIHH", 16, 3, 1, rate & 0xFFFFFFFF, (rate * 4) & 0xFFFFFFFF, 4, 32)
    head += b"data" + struct.pack("<I", n)
    return head + s.astype("<f4").tobytes()


def save(path: str, samples, sample_rate: float) -> None:
    """Write a 32-bit float mono WAV, atomically (write then rename)."""
    payload = wav_bytes(samples, sample_rate)
    d = os.path.dirname(os.path.abspath(path))
    fd, tmp = tempfile.mkstemp(dir=d, prefix=".wav-")
    try:
        with os.fdopen(fd, "wb") as fh:
            fh.write(payload)
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise
