"""Command line of the MI355X package (``src/trifusion_l4/cli.py``):
``info`` prints versions without touching the GPU; ``predict`` runs
``submission.run`` over a template directory with a local checkpoint."""

import argparse
from importlib import metadata
import json
from pathlib import Path
import platform

from . import __version__

DEPENDENCIES = ("torch", "numpy", "scipy", "soundfile", "einops")


def parser():
    p = argparse.ArgumentParser(prog="trifusion-amd")
    p.add_argument("--version", action="version", version=f"%(prog)s {__version__}")
    commands = p.add_subparsers(dest="command", required=True)
    commands.add_parser("info", help="Print installed versions without initializing the GPU")
    predict = commands.add_parser("predict", help="Run offline inference with your local checkpoint")
    predict.add_argument("--weights", type=Path, required=True)
    predict.add_argument("--root", type=Path, required=True, help="Directory containing data/ or open/")
    predict.add_argument("--graphs", action=argparse.BooleanOptionalAction, default=True)
    predict.add_argument("--padded-seconds", type=int, default=64)
    predict.add_argument("--max-batch", type=int, default=16)
    predict.add_argument("--workers", type=int, default=4)
    return p


def _versions():
    found = {}
    for name in DEPENDENCIES:
        try:
            found[name] = metadata.version(name)
        except metadata.PackageNotFoundError:
            found[name] = None
    return found


def main(argv=None):
    command = parser()
    args = command.parse_args(argv)
    if args.command == "info":
        info = {"version": __version__, "python": platform.python_version(), "platform": platform.system(),
                "dependencies": _versions()}
        print(json.dumps(info, indent=2))
        return 0
    if not args.weights.is_file():
        command.error(f"Checkpoint does not exist: {args.weights}")
    if not args.root.is_dir():
        command.error(f"Input root does not exist: {args.root}")
    if min(args.padded_seconds, args.max_batch, args.workers) < 1:
        command.error("Batch limits and worker count must be positive")
    from .submission import run

    run(args.root.resolve(), args.weights.resolve(), graphs=args.graphs, padded_seconds=args.padded_seconds,
        max_batch=args.max_batch, workers=args.workers)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
