"""Audio files -> padded 16 kHz batches for the MI355X engine.

Behaviour of ``src/trifusion_l4/audio.py``: every file is checked from its
header (1 or 2 channels, at most 72 s once resampled to 16 kHz), decoded to
float32, resampled to 16 kHz with ``scipy.signal.resample_poly`` (the exact
polyphase filter the reference uses), quantised to PCM16 and back, and grouped
by channel count and a length bucket (4 ... 72 s) into batches that stay under
a padded-seconds budget. Decoding runs on a thread pool with at most two
batches in flight; each batch is assembled in pinned host memory so the copy
to HBM can overlap the previous batch's forward.

WAV files (PCM 8/16/24/32-bit integer or IEEE float, plain or
WAVE_FORMAT_EXTENSIBLE) are parsed here. Other containers (FLAC, MP3, OGG,
M4A) go through ``soundfile`` when it is installed and raise otherwise.
"""

from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
import math
from pathlib import Path
import struct

import numpy as np
import torch

SAMPLE_RATE = 16000
MAX_SAMPLES = 72 * SAMPLE_RATE
BUCKET_SECONDS = (4, 8, 12, 16, 24, 32, 40, 48, 60, 72)

_PCM, _FLOAT, _EXTENSIBLE = 1, 3, 0xFFFE


@dataclass(frozen=True)
class AudioFile:
    index: int
    path: Path
    samples: int  # length at 16 kHz
    channels: int


@dataclass(frozen=True)
class _WavLayout:
    tag: int
    channels: int
    rate: int
    bits: int
    offset: int
    size: int

    @property
    def frames(self):
        return self.size // (self.channels * (self.bits // 8))


def _wav_layout(path):
    """Header of a RIFF/WAVE file: sample format, channels, rate, bit depth and
    the byte range of the sample data (the data itself is not read)."""
    with open(path, "rb") as f:
        head = f.read(12)
        if len(head) < 12 or head[:4] != b"RIFF" or head[8:12] != b"WAVE":
            raise ValueError(f"Not a RIFF/WAVE file: {path}")
        fmt = None
        while True:
            chunk = f.read(8)
            if len(chunk) < 8:
                raise ValueError(f"WAVE file without a data chunk: {path}")
            cid, size = chunk[:4], struct.unpack("<I", chunk[4:])[0]
            if cid == b"fmt ":
                body = f.read(size)
                if len(body) < 16:
                    raise ValueError(f"Truncated fmt chunk: {path}")
                tag, channels, rate, _, _, bits = struct.unpack("<HHIIHH", body[:16])
                if tag == _EXTENSIBLE:
                    if len(body) < 26:
                        raise ValueError(f"Truncated extensible fmt chunk: {path}")
                    tag = struct.unpack("<H", body[24:26])[0]  # first field of the sub-format GUID
                fmt = (tag, channels, rate, bits)
            elif cid == b"data":
                if fmt is None:
                    raise ValueError(f"WAVE data before fmt: {path}")
                offset = f.tell()
                f.seek(0, 2)
                size = min(size, f.tell() - offset)  # tolerate writers that leave the size unset
                layout = _WavLayout(*fmt, offset, size)
                if layout.tag not in (_PCM, _FLOAT) or layout.bits not in (
                    (8, 16, 24, 32) if layout.tag == _PCM else (32, 64)
                ):
                    raise ValueError(f"Unsupported WAVE sample format (tag {layout.tag}, {layout.bits} bits): {path}")
                if layout.channels < 1 or layout.rate < 1:
                    raise ValueError(f"Invalid WAVE header: {path}")
                return layout
            else:
                f.seek(size + (size & 1), 1)  # chunks are padded to even sizes
            if cid == b"fmt " and size & 1:
                f.seek(1, 1)


def _read_wav(path, layout):
    """float32 ``[frames, channels]`` normalised as libsndfile normalises: integer
    PCM divided by 2^(bits-1) (8-bit is unsigned, offset 128), floats as stored."""
    with open(path, "rb") as f:
        f.seek(layout.offset)
        raw = f.read(layout.frames * layout.channels * (layout.bits // 8))
    if layout.tag == _FLOAT:
        data = np.frombuffer(raw, dtype="<f4" if layout.bits == 32 else "<f8").astype(np.float32)
    elif layout.bits == 8:
        data = (np.frombuffer(raw, dtype=np.uint8).astype(np.float32) - 128.0) / 128.0
    elif layout.bits == 16:
        data = np.frombuffer(raw, dtype="<i2").astype(np.float32) / 32768.0
    elif layout.bits == 24:
        b = np.frombuffer(raw, dtype=np.uint8).reshape(-1, 3).astype(np.int32)
        v = b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16)
        v = np.where(v >= 1 << 23, v - (1 << 24), v)
        data = v.astype(np.float32) / 8388608.0
    else:
        data = (np.frombuffer(raw, dtype="<i4").astype(np.float64) / 2147483648.0).astype(np.float32)
    return data.reshape(-1, layout.channels)


def _soundfile():
    try:
        import soundfile
    except ModuleNotFoundError:
        return None
    return soundfile


def _is_wav(path):
    return Path(path).suffix.lower() == ".wav"


def _info(path):
    """(frames, rate, channels) from the file header."""
    if _is_wav(path):
        layout = _wav_layout(path)
        return layout.frames, layout.rate, layout.channels
    sf = _soundfile()
    if sf is None:
        raise ValueError(f"Decoding {Path(path).suffix} needs the soundfile package: {path}")
    info = sf.info(path)
    return info.frames, info.samplerate, info.channels


def _read(path):
    if _is_wav(path):
        layout = _wav_layout(path)
        return _read_wav(path, layout), layout.rate
    sf = _soundfile()
    if sf is None:
        raise ValueError(f"Decoding {Path(path).suffix} needs the soundfile package: {path}")
    return sf.read(path, dtype="float32", always_2d=True)


def inspect_audio(index, path):
    """``AudioFile`` from the header; the 16 kHz length is ceil(frames 16000 / rate)."""
    path = Path(path)
    frames, rate, channels = _info(path)
    samples = math.ceil(frames * SAMPLE_RATE / rate)
    if channels not in (1, 2) or not 0 < samples <= MAX_SAMPLES:
        raise ValueError(f"Unsupported audio dimensions: {path}")
    return AudioFile(index, path, samples, channels)


def decode_audio(record):
    """``[channels, samples]`` float32 tensor: decoded, resampled to 16 kHz,
    checked against the header, quantised to PCM16 and scaled back."""
    audio, rate = _read(record.path)
    if rate != SAMPLE_RATE:
        from scipy.signal import resample_poly

        g = math.gcd(rate, SAMPLE_RATE)
        audio = resample_poly(audio, SAMPLE_RATE // g, rate // g, axis=0).astype(np.float32)
    if audio.shape != (record.samples, record.channels) or not np.isfinite(audio).all():
        raise ValueError(f"Audio metadata or finite-value check failed: {record.path}")
    pcm = np.clip(np.rint(audio * 32768), -32768, 32767).astype(np.int16)
    return torch.from_numpy(np.ascontiguousarray((pcm.astype(np.float32) / 32768).T))


def bucket_limit(samples):
    """Padded length of a file: the smallest bucket of ``BUCKET_SECONDS`` that holds it."""
    for seconds in BUCKET_SECONDS:
        if samples <= seconds * SAMPLE_RATE:
            return seconds * SAMPLE_RATE
    raise ValueError(f"{samples} samples exceed the longest bucket")


def plan_batches(records, padded_seconds=120, max_batch=16, round_buckets=True):
    """``[(padded_length, [AudioFile, ...]), ...]``: files grouped by (channels,
    padded length), groups in sorted order, each cut into batches of
    max(1, min(max_batch, padded_seconds / padded_length)) files in input order.
    Without ``round_buckets`` every distinct length is its own group."""
    groups = {}
    for r in records:
        limit = bucket_limit(r.samples) if round_buckets else r.samples
        groups.setdefault((r.channels, limit), []).append(r)
    plan = []
    for (_, limit), rows in sorted(groups.items()):
        per = max(1, min(max_batch, int(padded_seconds * SAMPLE_RATE) // limit))
        plan.extend((limit, rows[i : i + per]) for i in range(0, len(rows), per))
    return plan


def decoded_batches(plan, workers=4):
    """Yield ``{"audio": [B, C, limit], "lengths": [B], "channels": [B], "indices": [...]}``
    per planned batch, decoding the next batch while the caller runs this one
    (never more than two batches of audio held)."""
    with ThreadPoolExecutor(max_workers=workers) as pool:
        batches = iter(plan)

        def start():
            item = next(batches, None)
            if item is None:
                return None
            limit, rows = item
            return limit, rows, [pool.submit(decode_audio, r) for r in rows]

        pending = start()
        while pending is not None:
            limit, rows, futures = pending
            pending = start()
            audio = torch.zeros(len(rows), rows[0].channels, limit, pin_memory=torch.cuda.is_available())
            for i, (record, future) in enumerate(zip(rows, futures)):
                audio[i, :, : record.samples] = future.result()
            yield {
                "audio": audio,
                "lengths": torch.tensor([r.samples for r in rows]),
                "channels": torch.tensor([r.channels for r in rows]),
                "indices": [r.index for r in rows],
            }
