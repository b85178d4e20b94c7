"""Collect the reference's golden grouping data as fixtures (data only).

Run once in the build container, where the reference is mounted read-only at
/root/reference; the GPU box never runs this script.  Writes
``tests/golden/grouping/<case>.state.npz`` (the input tick states, copied
byte for byte) and ``<case>.labels.npz`` (the expected 24 label arrays):

* the five bundled 4-player examples: ``asset/examples/4players/4_0k/``
  ``grouping_state.npz`` + ``groups.pt`` (the labels the reference's
  ``generate_labels`` must reproduce exactly, tests/test_dynamic_grouping.py:70-83);
* the three synthetic fixtures ``tests/fixtures/grouping/{p4_round_start,
  p6_moving_pairs,p10_moving_pairs}.{state,labels}.npz``
  (tests/test_dynamic_grouping.py:85-105).

``groups.pt`` is read with ``torch.load(weights_only=True)``; ``.npz`` files
with ``allow_pickle=False``.  No reference code is imported.

Usage: python tests/golden/make_grouping_golden.py [--ref /root/reference]
"""

from __future__ import annotations

import argparse
import csv
import shutil
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "grouping"
FIXTURES = ("p4_round_start", "p6_moving_pairs", "p10_moving_pairs")


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ref = Path(ap.parse_args().ref)
    OUT.mkdir(exist_ok=True)
    examples = ref / "asset/examples/4players"
    with open(examples / "metadata.csv", newline="") as fh:
        rows = list(csv.DictReader(fh))
    for row in rows:
        name = "example_" + Path(row["group_path"]).parent.name
        shutil.copyfile(examples / row["grouping_state_path"], OUT / f"{name}.state.npz")
        labels = torch.load(examples / row["group_path"], map_location="cpu", weights_only=True)
        np.savez_compressed(OUT / f"{name}.labels.npz", **{k: v.numpy() for k, v in labels.items()})
    for name in FIXTURES:
        src = ref / "tests/fixtures/grouping"
        shutil.copyfile(src / f"{name}.state.npz", OUT / f"{name}.state.npz")
        shutil.copyfile(src / f"{name}.labels.npz", OUT / f"{name}.labels.npz")
    print(f"wrote {len(rows) + len(FIXTURES)} cases to {OUT}")


if __name__ == "__main__":
    main()
