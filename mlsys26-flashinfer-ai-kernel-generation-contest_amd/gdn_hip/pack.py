"""Pack a solution directory into a flashinfer-bench Solution JSON.

Mirrors gdn_decode/scripts/pack_solution.py:34-82 (and the prefill variant's
destination_passing_style flag, gdn_prefill/scripts/pack_solution.py:56,61): the
metadata comes from ``solution/<name>/config.toml`` and the sources are the entry
``kernel.py`` plus everything it needs to build and run -- the ``gdn_hip`` package,
the HIP sources and the C ABI header -- as ``{"path", "content"}`` records in the
layout README.md:239-256 describes.

    python -m gdn_hip.pack gdn_decode [-o solution.json]
"""
from __future__ import annotations

import argparse
import glob
import json
import os
import sys

try:
    import tomllib  # Python >= 3.11
except ModuleNotFoundError:  # pragma: no cover - Python 3.10
    import tomli as tomllib

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
REPO = os.path.dirname(ROOT)


def _sources(solution_dir):
    files = [(os.path.join(solution_dir, "kernel.py"), "kernel.py")]
    for f in sorted(glob.glob(os.path.join(PKG_DIR, "*.py"))):
        files.append((f, "gdn_hip/" + os.path.basename(f)))
    for pat in ("*.hip", "*.h", "*.cpp"):
        for f in sorted(glob.glob(os.path.join(ROOT, "csrc", pat))):
            files.append((f, "csrc/" + os.path.basename(f)))
    files.append((os.path.join(REPO, "include", "gdn_hip.h"), "include/gdn_hip.h"))
    out = []
    for path, rel in files:
        with open(path) as fh:
            out.append({"path": rel, "content": fh.read()})
    return out


def pack_solution(name: str) -> dict:
    solution_dir = os.path.join(ROOT, "solution", name)
    cfg_path = os.path.join(solution_dir, "config.toml")
    if not os.path.exists(cfg_path):
        raise FileNotFoundError(f"config not found: {cfg_path}")
    with open(cfg_path, "rb") as fh:
        cfg = tomllib.load(fh)
    sol, bld = cfg["solution"], cfg["build"]
    return {
        "name": sol["name"],
        "definition": sol["definition"],
        "author": sol["author"],
        "spec": {
            "language": bld["language"],
            "target_hardware": bld.get("target_hardware", ["amd-mi355x"]),
            "entry_point": bld["entry_point"],
            "dependencies": [],
            "destination_passing_style": bool(bld.get("destination_passing_style", True)),
        },
        "sources": _sources(solution_dir),
    }


def main():
    ap = argparse.ArgumentParser(description="Pack a solution into solution JSON")
    ap.add_argument("name", choices=["gdn_decode", "gdn_prefill"])
    ap.add_argument("-o", "--output", default=None)
    args = ap.parse_args()
    doc = pack_solution(args.name)
    text = json.dumps(doc, indent=2)
    if args.output:
        with open(args.output, "w") as fh:
            fh.write(text)
        print(f"Solution packed: {args.output} ({doc['definition']}, {len(doc['sources'])} files)")
    else:
        sys.stdout.write(text)


if __name__ == "__main__":
    main()
