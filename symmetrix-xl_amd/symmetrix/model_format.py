"""Model files in both forms: the JSON v4 text the reference reads
(mace_kokkos_model.cpp) and SMXB, a binary form of the same document whose
number arrays are raw doubles (layout in csrc/model_binary.hpp).  Every
entry point that takes a model path accepts either form.

    python -m symmetrix.model_format model.json model.smxb           # JSON -> binary
    python -m symmetrix.model_format model.smxb model.json --format json
"""

from __future__ import annotations

import argparse
import os

from ._native import check, lib

MAGIC = b"SMXB"


def is_binary(path) -> bool:
    """True when the file starts with the SMXB magic."""
    with open(path, "rb") as f:
        return f.read(4) == MAGIC


def convert(source, destination, format="binary"):
    """Rewrite `source` (either form) as `format` ("binary" or "json") at
    `destination`; raises ValueError for a file that is not a format-4
    model, a corrupt binary file or an unknown format."""
    if format not in ("binary", "json"):
        raise ValueError("format must be 'binary' or 'json'")
    check(lib.smx_model_convert(os.fspath(source).encode(), os.fspath(destination).encode(), format.encode()))
    return destination


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("source")
    ap.add_argument("destination")
    ap.add_argument("--format", choices=("binary", "json"), default="binary")
    args = ap.parse_args(argv)
    convert(args.source, args.destination, args.format)


if __name__ == "__main__":
    main()
