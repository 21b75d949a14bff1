"""hipBLASLt solution choices for the ~1B decoder's projection GEMMs.

The decoder's dense layers (the q / k / v / o projections, the SwiGLU w1 / w3 / w2 and the tied LM
head, src/model/transformer.py and src/model/ffn.py) are plain library GEMMs through torch.
hipBLASLt's default heuristic picks a 256x256 macro-tile solution for the four shapes of a 16384-token
forward; timing every solution the library offers for those shapes (torch's TunableOp) finds one
that runs them at about 1.76 PFLOP/s.  ``data/tunableop_gfx950_decoder_1b.csv`` is that TunableOp
results file, written on an MI355X with this image's torch / HIP / hipBLASLt versions by

    PYTORCH_TUNABLEOP_ENABLED=1 PYTORCH_TUNABLEOP_TUNING=1 \\
    PYTORCH_TUNABLEOP_FILENAME=tunableop_results%d.csv \\
        python3 bench.py --workload decoder --steps 3 --warmup 2 --no-cpu-baseline

``use_tuned_gemms`` loads it with tuning switched off, so a forward only looks solutions up.  The
file's validator lines (torch, HIP and hipBLASLt versions, GPU arch) must match the running stack;
when they do not, the default heuristic stays in place.  The selection is a global torch setting:
it applies to every bf16 GEMM of these shapes in the process.
"""

from __future__ import annotations

import os
import tempfile

TUNED_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "tunableop_gfx950_decoder_1b.csv")


def tuned_shapes(path: str = TUNED_FILE) -> list:
    """The (op, shape, solution, ms) rows of a TunableOp results file (validator lines skipped)."""
    rows = []
    with open(path) as f:
        for line in f:
            parts = line.strip().split(",")
            if len(parts) == 4 and parts[0] != "Validator":
                rows.append((parts[0], parts[1], parts[2], float(parts[3])))
    return rows


def use_tuned_gemms(path: str = TUNED_FILE) -> str:
    """Switch torch's TunableOp on with the committed selections and tuning off; returns what the
    process now uses, for reporting.  Results TunableOp may write at exit go to a temporary file,
    never into the package."""
    import torch
    from torch.cuda import tunable

    if not torch.cuda.is_available():
        return "hipBLASLt default heuristic (no GPU)"
    if not os.path.exists(path):
        return "hipBLASLt default heuristic (no tuned file)"
    tunable.set_filename(os.path.join(tempfile.gettempdir(), f"pe_tunableop_{os.getpid()}.csv"))
    tunable.tuning_enable(False)
    tunable.enable(True)
    if not tunable.read_file(path):
        tunable.enable(False)
        return "hipBLASLt default heuristic (tuned file not accepted by this torch / hipBLASLt)"
    return f"torch TunableOp selections from {os.path.relpath(path, os.path.dirname(os.path.dirname(os.path.dirname(path))))}"
