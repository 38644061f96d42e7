"""The submission CSV contract, with no GPU or model imports.

Behaviour of ``src/trifusion_l4/submission_format.py``: the one
``sample_submission.csv`` under ``<root>/data`` or ``<root>/open`` fixes the
output columns (their order, and the ID of every row); each of the five outputs
maps to exactly one column named ``<output>`` or ``<output>_PROB`` (case
insensitive); every ID maps to exactly one audio file under the same data
directory, by file name, stem or relative path. Predictions are written in the
template's row and column order, as ``.9g`` decimals, through a temporary file
renamed into place, so an invalid prediction set never leaves an output.
"""

import csv
import math
from pathlib import Path

OUTPUTS = ("file_fake", "voice_fake", "music_fake", "voice_present", "music_present")
AUDIO_SUFFIXES = (".wav", ".flac", ".mp3", ".ogg", ".m4a")
DATA_DIRS = ("data", "open")


def _template(root):
    found = []
    for name in DATA_DIRS:
        directory = Path(root) / name
        if directory.exists():
            found.extend(directory.rglob("sample_submission.csv"))
    if len(found) != 1:
        raise ValueError(f"Expected one official sample_submission.csv; found {len(found)}")
    return found[0]


def _output_columns(columns):
    aliases = {}
    for name in OUTPUTS:
        hits = [c for c in columns if c.casefold() in (name, name + "_prob")]
        if len(hits) != 1:
            raise ValueError(f"Expected one output column for {name}; found {hits}")
        aliases[name] = hits[0]
    rest = [c for c in columns if c not in aliases.values()]
    if len(rest) != 1 or rest[0].casefold() != "id":
        raise ValueError("Template must have exactly one ID column")
    return aliases, rest[0]


def _audio_index(data_root):
    index = {}
    for path in data_root.rglob("*"):
        if path.is_file() and path.suffix.lower() in AUDIO_SUFFIXES:
            for key in {path.name, path.stem, str(path.relative_to(data_root))}:
                index.setdefault(key, set()).add(path)
    return index


def discover_inputs(root):
    """``(columns, rows, aliases, paths)``: the template's header, its rows as
    dicts (IDs stripped), output name -> column, and the audio file of each row."""
    template = _template(root)
    with template.open(newline="", encoding="utf-8-sig") as f:
        reader = csv.DictReader(f)
        columns = reader.fieldnames
        rows = list(reader)
    if not columns or not rows:
        raise ValueError("Empty submission template")
    if len({c.casefold() for c in columns}) != len(columns):
        raise ValueError("Duplicate template columns")
    aliases, id_column = _output_columns(columns)
    ids = []
    for row in rows:
        value = (row.get(id_column) or "").strip()
        if not value:
            raise ValueError("Empty template ID")
        row[id_column] = value
        ids.append(value)
    if len(set(ids)) != len(ids):
        raise ValueError("Duplicate template IDs")
    data_root = next(Path(root) / n for n in DATA_DIRS if Path(root) / n in template.parents)
    index = _audio_index(data_root)
    paths = []
    for value in ids:
        hits = index.get(value, set())
        if len(hits) != 1:
            raise ValueError(f"Expected one audio file for ID {value!r}; found {len(hits)}")
        paths.append(next(iter(hits)))
    return columns, rows, aliases, paths


def write_submission(path, columns, rows, aliases, predictions):
    """Write one row per template row with its five probabilities (finite, in
    [0, 1]) in the output columns; other cells keep the template's values."""
    predictions = [tuple(float(v) for v in row) for row in predictions]
    valid = len(predictions) == len(rows) and all(
        len(row) == len(OUTPUTS) and all(math.isfinite(v) and 0.0 <= v <= 1.0 for v in row) for row in predictions
    )
    if not valid:
        raise ValueError("Predictions must be finite [0,1] values for every template row")
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    partial = path.with_suffix(".partial")
    with partial.open("w", newline="", encoding="utf-8") as f:
        writer = csv.DictWriter(f, fieldnames=columns)
        writer.writeheader()
        for row, values in zip(rows, predictions):
            out = dict(row)
            out.update({aliases[name]: format(v, ".9g") for name, v in zip(OUTPUTS, values)})
            writer.writerow(out)
    partial.replace(path)
