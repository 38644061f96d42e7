"""``trifusion-amd`` command line.

Two commands, with the subcommand names and flags of the reference's
``trifusion-l4`` (src/trifusion_l4/cli.py:12-25, pyproject.toml:42-43):

* ``info`` prints a JSON description of the installation: package version,
  Python, OS, dependency versions and whether the native library is built.
  It imports neither torch nor the library, so it never opens a GPU.
* ``predict --weights W --root R`` writes ``R/output/submission.csv`` and
  ``R/output/runtime_report.json`` (see ``submission.run``).

Flag values are checked while they are parsed (``type=`` converters), so a
bad value exits with status 2 and names its flag before any model, audio or
GPU work starts.
"""

import argparse
from importlib import metadata
import json
from pathlib import Path
import platform

from . import __version__

DEPENDENCIES = ("torch", "numpy", "scipy", "soundfile", "einops")
LIBRARY = Path(__file__).with_name("libtrifusion_amd.so")


def _file(text):
    path = Path(text)
    if not path.is_file():
        raise argparse.ArgumentTypeError(f"no checkpoint file at {text}")
    return path.resolve()


def _directory(text):
    path = Path(text)
    if not path.is_dir():
        raise argparse.ArgumentTypeError(f"{text} is not a directory")
    return path.resolve()


def _count(text):
    try:
        value = int(text)
    except ValueError:
        raise argparse.ArgumentTypeError(f"{text!r} is not an integer") from None
    if value < 1:
        raise argparse.ArgumentTypeError(f"{value} is too small (the least accepted value is 1)")
    return value


def _installed(name):
    try:
        return metadata.version(name)
    except metadata.PackageNotFoundError:
        return None


def info(_args):
    report = {
        "version": __version__,
        "python": platform.python_version(),
        "platform": platform.system(),
        "dependencies": {name: _installed(name) for name in DEPENDENCIES},
        "native_library": str(LIBRARY) if LIBRARY.exists() else None,
    }
    print(json.dumps(report, indent=2))
    return 0


def predict(args):
    from .submission import run

    run(args.root, args.weights, graphs=args.graphs, padded_seconds=args.padded_seconds,
        max_batch=args.max_batch, workers=args.workers)
    return 0


def _predict_flags(sub):
    sub.add_argument("--weights", type=_file, required=True, metavar="CHECKPOINT",
                     help="student checkpoint written by runtime.save_student")
    sub.add_argument("--root", type=_directory, required=True,
                     help="dataset folder; its data/ or open/ subfolder holds sample_submission.csv and the audio")
    sub.add_argument("--graphs", action=argparse.BooleanOptionalAction, default=True,
                     help="replay one captured HIP graph per length bucket (--no-graphs: eager launches)")
    sub.add_argument("--padded-seconds", type=_count, default=64,
                     help="longest padded clip, in seconds, that a batch may hold")
    sub.add_argument("--max-batch", type=_count, default=16, help="most clips per batch")
    sub.add_argument("--workers", type=_count, default=4, help="audio decoding threads")


COMMANDS = {
    "info": ("describe the installation as JSON (opens no GPU)", None, info),
    "predict": ("score every row of a submission template on the GPU", _predict_flags, predict),
}


def parser():
    top = argparse.ArgumentParser(prog="trifusion-amd", description="TriFusion-FP inference on AMD Instinct MI355X")
    top.add_argument("--version", action="version", version=f"%(prog)s {__version__}")
    subs = top.add_subparsers(dest="command", required=True, metavar="COMMAND")
    for name, (summary, flags, handler) in COMMANDS.items():
        sub = subs.add_parser(name, help=summary, description=summary)
        if flags is not None:
            flags(sub)
        sub.set_defaults(handler=handler)
    return top


def main(argv=None):
    args = parser().parse_args(argv)
    return args.handler(args)


if __name__ == "__main__":
    raise SystemExit(main())
