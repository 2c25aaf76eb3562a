"""Quantize an exported model (and its drafters) to the FP8 checkpoint that
``--precision fp8`` serves: the CLI of ``export_fp8.py:15-44`` over this
package's quantizer.

    python -m jeeves_amd.export_fp8 EXPORT_DIR --out OUT [--drafter FILE ...] [--linears NAMES.json] [--force]

Which linears to quantize: by default the jeeves model's own list (its
``meta_view`` + ``quantized_linears``; needs the jeeves tree importable, as
``load_view`` does); ``--linears`` takes a JSON list of module names instead
(base-model linears prefixed ``base.``, drafter linears without prefix, as in
the reference's drafter view). The output has the same layout as the
reference's: quantized shards under the input shard names, a rewritten
``model.safetensors.index.json``, the drafters under their file names, the
other files copied, and ``export.json`` with ``"precision": "fp8"``.
"""

from __future__ import annotations

import argparse
import json
import shutil
import sys
from pathlib import Path

from .fp8_checkpoint import write_quantized

BASE = "base."
INDEX = "model.safetensors.index.json"
# Files rewritten here rather than copied (export_fp8.py:12).
NOT_COPIED = {INDEX, "export.json", "README.md", ".gitattributes"}


def model_linears(src: Path) -> set[str]:
    """The jeeves model's quantizable linears (needs its tree on sys.path)."""
    try:
        from inference.fp8_checkpoint import meta_view, quantized_linears
        from model import Qwen3_5_9BConfig
    except ImportError as e:
        raise SystemExit("without --linears the jeeves model code must be importable (run from the jeeves tree)") from e
    return quantized_linears(meta_view(Qwen3_5_9BConfig.from_json(src / "config.json")))


def export(src: Path, out: Path, linears: set[str], drafters: list[Path], force: bool = False) -> dict:
    """Write the FP8 export of ``src`` to ``out``; returns the summary the CLI prints."""
    if len({d.name for d in drafters}) < len(drafters):
        raise ValueError(f"drafters are written to --out under their file names, which must differ: {drafters}")
    if out.exists() and any(out.iterdir()) and not force:
        raise FileExistsError(f"{out} is not empty; pass --force")
    out.mkdir(parents=True, exist_ok=True)
    base = {n[len(BASE):] for n in linears if n.startswith(BASE)}
    drafter_linears = {n for n in linears if not n.startswith(BASE)}
    shards = sorted(set(json.loads((src / INDEX).read_text())["weight_map"].values()))
    weight_map: dict[str, str] = {}
    total = 0
    for shard in shards:
        sizes = write_quantized(src / shard, out / shard, base)
        weight_map.update({key: shard for key in sizes})
        total += sum(sizes.values())
    (out / INDEX).write_text(json.dumps({"metadata": {"total_size": total}, "weight_map": weight_map}, indent=2) + "\n")
    for drafter in drafters:
        total += sum(write_quantized(drafter, out / drafter.name, drafter_linears).values())
    for f in src.iterdir():
        if f.is_file() and f.suffix != ".safetensors" and f.name not in NOT_COPIED:
            shutil.copyfile(f, out / f.name)
    meta = json.loads((src / "export.json").read_text()) if (src / "export.json").exists() else {}
    meta["precision"] = "fp8"
    (out / "export.json").write_text(json.dumps(meta, indent=2) + "\n")
    return {"out": str(out), "quantized_linears": len(linears), "drafters": len(drafters), "total_gb": round(total / 2**30, 2)}


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser(description="Quantize an exported model and its drafters to the FP8 weights that "
                                             "--precision fp8 serves.")
    ap.add_argument("model", help="export directory")
    ap.add_argument("--drafter", action="append", default=[], help="drafter safetensors to quantize into --out; repeat for more")
    ap.add_argument("--out", required=True)
    ap.add_argument("--linears", help="JSON list of linear module names to quantize (default: the jeeves model's)")
    ap.add_argument("--force", action="store_true")
    a = ap.parse_args(argv)
    src = Path(a.model)
    linears = set(json.loads(Path(a.linears).read_text())) if a.linears else model_linears(src)
    print(json.dumps(export(src, Path(a.out), linears, [Path(d) for d in a.drafter], a.force)))


if __name__ == "__main__":
    sys.exit(main())
