"""Copy the reference's own recorded golden data for this path into tests/golden/.

Run in the build container only (it reads /root/reference); its outputs are committed
and the tests read those, never the reference.  Nothing from the reference is imported
or executed: the cards are text files and the verify table is JSON.

Sources:
  bench/results/e1/2026-08-28_131651-runpod-nvidia/lanes/gemm.identical.card
      host oracle card, 20 shapes capped to 16M MACs (bench/gemm_card_main.mojo:238-241,361-378)
  bench/results/amd_step_time_2026-09-24/legs/2026-09-24_234736-do-mi325x/remote/amd.card
      MI325X device card, the same 20 shapes capped to 64Mi device floats
  bench/results/e1g/2026-09-17_203449-nvidia-refregen-par-lanes-b/remote/nvidia.card
      NVIDIA device card (byte-identical fields 2-5 to the MI325X one)
  python/mojolearn/verify_reference/table.json
      cells gemm-pinned/*, gemm-transposed/*, gemm-bf16/*, gemm-int8/*, gemm-int15/*, lowbit-conversions/*
      (train column) and the
      fixture X hashes (tools/identity_break.py:1355-1382 hashing, :1434-1509 fixtures)
"""
import json
import os
import shutil

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))

CARDS = {
    "host_oracle.card": "bench/results/e1/2026-08-28_131651-runpod-nvidia/lanes/gemm.identical.card",
    "device_mi325x.card": "bench/results/amd_step_time_2026-09-24/legs/2026-09-24_234736-do-mi325x/remote/amd.card",
    "device_nvidia.card": "bench/results/e1g/2026-09-17_203449-nvidia-refregen-par-lanes-b/remote/nvidia.card",
}


def main():
    os.makedirs(os.path.join(HERE, "cards"), exist_ok=True)
    for dst, src in CARDS.items():
        shutil.copyfile(os.path.join(REF, src), os.path.join(HERE, "cards", dst))
    with open(os.path.join(REF, "python/mojolearn/verify_reference/table.json")) as fh:
        table = json.load(fh)
    cells = {}
    for name, cell in table["cells"].items():
        lane = name.split("/")[0]
        if lane in ("gemm-pinned", "gemm-transposed", "gemm-bf16", "gemm-int8", "gemm-int15", "lowbit-conversions"):
            cells[name] = {"train": cell["train"]["ref"]}
    out = {
        "source": "python/mojolearn/verify_reference/table.json",
        "format": table["format"],
        "fixtures": {k: v["X"] for k, v in table["fixtures"].items()},
        "cells": dict(sorted(cells.items())),
    }
    with open(os.path.join(HERE, "verify_gemm_cells.json"), "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
        fh.write("\n")


if __name__ == "__main__":
    main()
