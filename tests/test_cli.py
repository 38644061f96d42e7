"""Command line (no GPU): ``info`` reports versions without initialising the
GPU, ``predict`` validates its arguments before loading anything."""

import json

import pytest

from trifusion_amd import __version__, cli


def test_info_reports_versions(capsys):
    assert cli.main(["info"]) == 0
    info = json.loads(capsys.readouterr().out)
    assert info["version"] == __version__ and set(info["dependencies"]) == set(cli.DEPENDENCIES)


def test_version_flag(capsys):
    with pytest.raises(SystemExit) as e:
        cli.main(["--version"])
    assert e.value.code == 0 and __version__ in capsys.readouterr().out


@pytest.mark.parametrize("case", ["no-weights", "no-root", "zero-batch"])
def test_predict_rejects_bad_arguments(tmp_path, capsys, case):
    weights = tmp_path / "w.pt"
    weights.write_bytes(b"x")
    args = ["predict", "--weights", str(weights), "--root", str(tmp_path)]
    if case == "no-weights":
        args[2] = str(tmp_path / "missing.pt")
    elif case == "no-root":
        args[4] = str(tmp_path / "missing")
    else:
        args += ["--max-batch", "0"]
    with pytest.raises(SystemExit) as e:
        cli.main(args)
    assert e.value.code == 2
    message = capsys.readouterr().err
    assert {"no-weights": "Checkpoint", "no-root": "Input root", "zero-batch": "positive"}[case] in message
