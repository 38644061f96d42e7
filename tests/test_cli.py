"""Command line (no GPU): ``info`` reports versions without initialising the
GPU, ``predict`` rejects bad flag values while parsing, naming the flag,
before loading anything."""

import json
import sys

import pytest

from trifusion_amd import __version__, cli


def test_info_reports_versions(capsys):
    assert cli.main(["info"]) == 0
    info = json.loads(capsys.readouterr().out)
    assert info["version"] == __version__ and set(info["dependencies"]) == set(cli.DEPENDENCIES)
    assert set(info) == {"version", "python", "platform", "dependencies", "native_library"}


def test_info_opens_no_gpu():
    """``info`` must not import torch (which would bring up the HIP runtime)."""
    import os
    import subprocess

    package = os.path.dirname(os.path.dirname(cli.__file__))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(filter(None, [package, os.environ.get("PYTHONPATH")])))
    code = "import sys; from trifusion_amd import cli; cli.main(['info']); print('torch' in sys.modules)"
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True, env=env).stdout
    assert out.strip().splitlines()[-1] == "False"


def test_version_flag(capsys):
    with pytest.raises(SystemExit) as e:
        cli.main(["--version"])
    assert e.value.code == 0 and __version__ in capsys.readouterr().out


@pytest.mark.parametrize("case", ["no-weights", "no-root", "zero-batch", "text-workers", "negative-seconds"])
def test_predict_rejects_bad_arguments(tmp_path, capsys, case):
    weights = tmp_path / "w.pt"
    weights.write_bytes(b"x")
    args = ["predict", "--weights", str(weights), "--root", str(tmp_path)]
    if case == "no-weights":
        args[2] = str(tmp_path / "missing.pt")
    elif case == "no-root":
        args[4] = str(tmp_path / "missing")
    elif case == "zero-batch":
        args += ["--max-batch", "0"]
    elif case == "text-workers":
        args += ["--workers", "four"]
    else:
        args += ["--padded-seconds", "-3"]
    with pytest.raises(SystemExit) as e:
        cli.main(args)
    assert e.value.code == 2
    message = capsys.readouterr().err
    flag, reason = {"no-weights": ("--weights", "no checkpoint file"), "no-root": ("--root", "not a directory"),
                    "zero-batch": ("--max-batch", "least accepted value is 1"),
                    "text-workers": ("--workers", "not an integer"),
                    "negative-seconds": ("--padded-seconds", "least accepted value is 1")}[case]
    assert flag in message and reason in message


def test_predict_parses_defaults(tmp_path):
    weights = tmp_path / "w.pt"
    weights.write_bytes(b"x")
    args = cli.parser().parse_args(["predict", "--weights", str(weights), "--root", str(tmp_path), "--no-graphs"])
    assert (args.graphs, args.padded_seconds, args.max_batch, args.workers) == (False, 64, 16, 4)
    assert args.weights == weights.resolve() and args.root == tmp_path.resolve()
    assert args.handler is cli.predict
