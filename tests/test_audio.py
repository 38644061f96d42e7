"""Audio decoding, resampling, quantisation and batch planning (no GPU).
WAV fixtures are written with the standard library's ``wave`` writer (integer
PCM) and by hand (IEEE float, WAVE_FORMAT_EXTENSIBLE), so the parser is checked
against independently produced files; resampling is checked against
``scipy.signal.resample_poly`` followed by the PCM16 round trip, as the
reference's own test does (tests/test_submission.py)."""

import struct
import wave

import numpy as np
import pytest
import torch
from scipy.signal import resample_poly

from trifusion_amd.audio import (
    MAX_SAMPLES,
    SAMPLE_RATE,
    AudioFile,
    decode_audio,
    decoded_batches,
    inspect_audio,
    plan_batches,
)


def write_pcm(path, ints, rate, width):
    """Integer PCM through the stdlib writer; ints [frames, channels]."""
    ints = np.asarray(ints)
    if width == 1:
        raw = (ints + 128).astype(np.uint8).tobytes()
    elif width == 3:
        v = ints.astype(np.int64).reshape(-1) & 0xFFFFFF
        raw = np.stack([(v >> s) & 0xFF for s in (0, 8, 16)], -1).astype(np.uint8).tobytes()
    else:
        raw = ints.astype({2: "<i2", 4: "<i4"}[width]).tobytes()
    with wave.open(str(path), "wb") as w:
        w.setnchannels(ints.shape[1])
        w.setsampwidth(width)
        w.setframerate(rate)
        w.writeframes(raw)


def write_float(path, data, rate, extensible=False, bits=32):
    """IEEE-float WAVE written field by field; optionally the extensible header."""
    data = np.asarray(data, dtype="<f4" if bits == 32 else "<f8")
    ch = data.shape[1]
    block = ch * bits // 8
    if extensible:
        guid = struct.pack("<H", 3) + bytes.fromhex("000000001000800000aa00389b71")
        fmt = struct.pack("<HHIIHHHHI", 0xFFFE, ch, rate, rate * block, block, bits, 22, bits, 0) + guid
    else:
        fmt = struct.pack("<HHIIHH", 3, ch, rate, rate * block, block, bits)
    body = data.tobytes()
    chunks = b"fmt " + struct.pack("<I", len(fmt)) + fmt
    chunks += b"LIST" + struct.pack("<I", 5) + b"abcde\0"  # odd-sized chunk before the data
    chunks += b"data" + struct.pack("<I", len(body)) + body
    path.write_bytes(b"RIFF" + struct.pack("<I", 4 + len(chunks)) + b"WAVE" + chunks)


def quantised(x):
    return np.clip(np.rint(x * 32768), -32768, 32767).astype(np.int16).astype(np.float32) / 32768


@pytest.mark.parametrize("width,scale", [(1, 128.0), (2, 32768.0), (3, 8388608.0), (4, 2147483648.0)])
def test_integer_pcm_is_normalised_by_its_width(tmp_path, width, scale):
    rng = np.random.default_rng(width)
    top = int(scale)
    ints = rng.integers(-top, top, (3000, 2))
    path = tmp_path / f"pcm{width}.wav"
    write_pcm(path, ints, SAMPLE_RATE, width)
    record = inspect_audio(5, path)
    assert record == AudioFile(5, path, 3000, 2)
    out = decode_audio(record).numpy()
    assert out.shape == (2, 3000)
    np.testing.assert_array_equal(out, quantised((ints / scale).astype(np.float32)).T)


@pytest.mark.parametrize("extensible", [False, True])
@pytest.mark.parametrize("bits", [32, 64])
def test_float_wav_resampled_and_quantised(tmp_path, extensible, bits):
    rng = np.random.default_rng(77)
    source = rng.normal(0, 0.1, (44100, 2)).astype(np.float32)
    path = tmp_path / "stereo.wav"
    write_float(path, source, 44100, extensible, bits)
    record = inspect_audio(0, path)
    assert record.samples == 16000 and record.channels == 2
    expected = quantised(resample_poly(source, 160, 441, axis=0).astype(np.float32))
    np.testing.assert_array_equal(decode_audio(record).numpy().T, expected)


def test_dimension_limits(tmp_path):
    write_pcm(tmp_path / "three.wav", np.zeros((100, 3), dtype=np.int64), SAMPLE_RATE, 2)
    write_pcm(tmp_path / "empty.wav", np.zeros((0, 1), dtype=np.int64), SAMPLE_RATE, 2)
    write_pcm(tmp_path / "long.wav", np.zeros((MAX_SAMPLES // 2 + 1, 1), dtype=np.int64), SAMPLE_RATE // 2, 2)
    for name in ("three.wav", "empty.wav", "long.wav"):
        with pytest.raises(ValueError, match="Unsupported audio dimensions"):
            inspect_audio(0, tmp_path / name)
    (tmp_path / "bad.wav").write_bytes(b"RIFX0000WAVE")
    with pytest.raises(ValueError, match="RIFF"):
        inspect_audio(0, tmp_path / "bad.wav")


def test_nonfinite_audio_is_rejected(tmp_path):
    data = np.zeros((100, 1), dtype=np.float32)
    data[7] = np.nan
    write_float(tmp_path / "nan.wav", data, SAMPLE_RATE)
    with pytest.raises(ValueError, match="finite"):
        decode_audio(inspect_audio(0, tmp_path / "nan.wav"))


def test_other_containers_need_soundfile(tmp_path, monkeypatch):
    import trifusion_amd.audio as A

    monkeypatch.setattr(A, "_soundfile", lambda: None)
    (tmp_path / "x.flac").write_bytes(b"fLaC")
    with pytest.raises(ValueError, match="soundfile"):
        inspect_audio(0, tmp_path / "x.flac")


def test_plan_groups_by_channels_and_bucket():
    records = [AudioFile(i, None, n, c) for i, (n, c) in enumerate(
        [(16001, 1), (64000, 1), (64001, 1), (10, 2), (64000, 1), (1_000_000, 1), (64000, 1)])]
    plan = plan_batches(records, padded_seconds=12, max_batch=2)
    # mono 4 s: 12 s // 4 s = 3 per batch, capped at 2; 8 s and 72 s: 1 per batch; stereo last
    assert [(limit, [r.index for r in rows]) for limit, rows in plan] == [
        (4 * SAMPLE_RATE, [0, 1]), (4 * SAMPLE_RATE, [4, 6]), (8 * SAMPLE_RATE, [2]), (72 * SAMPLE_RATE, [5]),
        (4 * SAMPLE_RATE, [3])]
    exact = plan_batches(records, padded_seconds=12, max_batch=16, round_buckets=False)
    assert {limit for limit, _ in exact} == {16001, 64000, 64001, 10, 1_000_000}
    assert [r.index for limit, rows in exact if limit == 64000 for r in rows] == [1, 4, 6]


def test_decoded_batches_pad_and_keep_indices(tmp_path):
    lengths = [16001, 32000, 64001]
    records = []
    for i, n in enumerate(lengths):
        ints = np.random.default_rng(i).integers(-3000, 3000, (n, 1))
        write_pcm(tmp_path / f"{i}.wav", ints, SAMPLE_RATE, 2)
        records.append(inspect_audio(i, tmp_path / f"{i}.wav"))
    seen = []
    for batch in decoded_batches(plan_batches(records, 4, 2), workers=2):
        audio = batch["audio"]
        for row, (i, n) in enumerate(zip(batch["indices"], batch["lengths"].tolist())):
            assert n == lengths[i]
            assert torch.equal(audio[row, :, :n], decode_audio(records[i]))
            assert not audio[row, :, n:].any()
        assert batch["channels"].tolist() == [1] * len(batch["indices"])
        seen += batch["indices"]
    assert sorted(seen) == [0, 1, 2]
