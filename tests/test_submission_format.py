"""The submission CSV contract (no GPU): template discovery, output column
aliases, ID normalisation and audio mapping, and all-or-nothing writes. Cases
follow the reference's own contract tests (tests/test_submission_format.py)."""

import csv

import pytest

from trifusion_amd.submission_format import discover_inputs, write_submission

OFFICIAL = ["ID", "FILE_FAKE_PROB", "VOICE_FAKE_PROB", "MUSIC_FAKE_PROB", "VOICE_PRESENT_PROB", "MUSIC_PRESENT_PROB"]


@pytest.fixture
def root(tmp_path):
    (tmp_path / "data/test").mkdir(parents=True)
    for name in ("TEST_0000.wav", "TEST_0001.mp3", "TEST_0002.flac"):
        (tmp_path / "data/test" / name).touch()
    return tmp_path


def template(root, columns=OFFICIAL, ids=("TEST_0002", "TEST_0000", "TEST_0001")):
    with (root / "data/sample_submission.csv").open("w", encoding="utf-8-sig", newline="") as f:
        w = csv.DictWriter(f, fieldnames=columns)
        w.writeheader()
        for value in ids:
            w.writerow({**dict.fromkeys(columns, 0), "ID": value})


def read(path):
    with path.open() as f:
        reader = csv.DictReader(f)
        return reader.fieldnames, list(reader)


def test_template_order_and_probability_mapping(root):
    template(root)
    columns, rows, aliases, paths = discover_inputs(root)
    assert [p.name for p in paths] == ["TEST_0002.flac", "TEST_0000.wav", "TEST_0001.mp3"]
    predictions = [[0.1, 0.2, 0.3, 0.4, 0.5], [0.9, 0.8, 0.7, 0.6, 0.5], [0, 1, 0, 1, 0]]
    write_submission(root / "output/submission.csv", columns, rows, aliases, predictions)
    header, out = read(root / "output/submission.csv")
    assert header == OFFICIAL
    assert [r["ID"] for r in out] == ["TEST_0002", "TEST_0000", "TEST_0001"]
    assert [float(out[0][c]) for c in OFFICIAL[1:]] == [0.1, 0.2, 0.3, 0.4, 0.5]


def test_column_order_of_the_template_is_kept(root):
    order = ["ID", "VOICE_PRESENT_PROB", "MUSIC_FAKE_PROB", "FILE_FAKE_PROB", "MUSIC_PRESENT_PROB", "VOICE_FAKE_PROB"]
    template(root, order)
    columns, rows, aliases, _ = discover_inputs(root)
    write_submission(root / "out.csv", columns, rows, aliases, [[0.1, 0.2, 0.3, 0.4, 0.5]] * 3)
    header, out = read(root / "out.csv")
    assert header == order
    assert float(out[0]["VOICE_PRESENT_PROB"]) == 0.4 and float(out[0]["VOICE_FAKE_PROB"]) == 0.2


def test_unsuffixed_columns_are_accepted(root):
    columns = [c.replace("_PROB", "") for c in OFFICIAL]
    template(root, columns)
    actual, _, aliases, _ = discover_inputs(root)
    assert actual == columns and aliases["voice_fake"] == "VOICE_FAKE"


@pytest.mark.parametrize("columns", [OFFICIAL[:-1], OFFICIAL + ["VOICE_FAKE"], OFFICIAL + ["FILE_FAKE_PROB"]])
def test_missing_or_ambiguous_output_columns_fail(root, columns):
    template(root, columns)
    with pytest.raises(ValueError):
        discover_inputs(root)


def test_ids_are_stripped_and_must_be_unique_and_present(root):
    template(root, ids=[" TEST_0000 ", "TEST_0001", "TEST_0002"])
    assert discover_inputs(root)[1][0]["ID"] == "TEST_0000"
    for ids in (["TEST_0000", " TEST_0000 "], ["TEST_0000", " "]):
        template(root, ids=ids)
        with pytest.raises(ValueError):
            discover_inputs(root)


def test_missing_or_ambiguous_audio_fails(root):
    template(root, ids=["UNKNOWN"])
    with pytest.raises(ValueError, match="Expected one audio"):
        discover_inputs(root)
    template(root)
    (root / "data/test/TEST_0000.flac").touch()
    with pytest.raises(ValueError, match="Expected one audio"):
        discover_inputs(root)


def test_one_template_is_required(root):
    with pytest.raises(ValueError, match="sample_submission"):
        discover_inputs(root)
    template(root)
    (root / "open").mkdir()
    (root / "open/sample_submission.csv").write_text((root / "data/sample_submission.csv").read_text())
    with pytest.raises(ValueError, match="found 2"):
        discover_inputs(root)


@pytest.mark.parametrize("predictions", [[], [[0.2] * 4] * 3, [[float("nan")] * 5] * 3, [[float("inf")] * 5] * 3,
                                         [[-0.1] * 5] * 3, [[1.1] * 5] * 3])
def test_invalid_predictions_leave_no_output(root, predictions):
    template(root)
    columns, rows, aliases, _ = discover_inputs(root)
    with pytest.raises(ValueError, match="finite"):
        write_submission(root / "out.csv", columns, rows, aliases, predictions)
    assert not (root / "out.csv").exists() and not (root / "out.partial").exists()
