"""Long-context perplexity harness: drop-in for scripts/evaluate_long_context.py.

``load_model`` reads a checkpoint in the reference trainer's format (src/training/trainer.py:
203-214: ``model_state_dict``, ``model_config`` as a plain dict, optionally ``config``) into this
library's ``Transformer`` (scripts/evaluate_long_context.py:28-69), and
``compute_ppl_sliding_window`` is the reference's windowed loop (:80-137) with its exact
accounting: windows of ``context_length`` tokens every ``stride`` (default half a window) over the
first ``4 * context_length`` tokens, each window's mean next-token loss weighted by
``context_length // 2``, stopping once ``2 * context_length`` tokens are counted, and
``(inf, True)`` on an out-of-memory error.  Every attention layer runs the library's fused HIP
kernel.

Differences from the reference script, all at the I/O edge:
- checkpoints are read with ``torch.load(weights_only=True)`` (the trainer's checkpoint holds
  only tensors, numbers, strings and dicts of them, so nothing has to be unpickled as code);
- the token stream comes from a file (``--tokens``: ``.npy`` of integer ids, or text of
  whitespace-separated ids), since this build has no dataset download or tokenizer;
- ``--dtype bf16`` optionally runs the model in bf16 (the reference evaluates in fp32, the default).

CLI: python -m pe_ablations_amd.evaluation --checkpoint-dir DIR --tokens FILE
         [--context-lengths 512 1024 ...] [--output-dir DIR] [--device cuda:0] [--models ...]
"""

from __future__ import annotations

import argparse
import gc
import json
import math
from pathlib import Path
from typing import Optional, Sequence

import torch

from .transformer import Transformer, TransformerConfig

# model_config keys the reference script reads, with its defaults (scripts/evaluate_long_context.py:35-59)
_CONFIG_KEYS = {
    "vocab_size": 50257, "hidden_dim": 512, "num_layers": 24, "num_heads": 8, "num_kv_heads": 4,
    "head_dim": 64, "max_seq_len": 512, "pe_mode": "rope",
    "rope_theta": 10000.0, "rope_type": "standard", "rope_scale": 1.0,
    "fpope_theta": 10000.0, "fpope_num_fourier_terms": 64, "fpope_sigma": 0.4,
    "fpope_training_length": 512, "fpope_delta_init": "zero", "fpope_d_rope": 32,
    "fpope_freeze_coeffs": False, "fpope_use_ceiling": False, "fpope_normalize_coeffs": True,
    "pope_theta": 10000.0, "pope_training_length": 512, "pope_delta_init": "zero", "pope_d_rope": 32,
}


# read in addition: both only turn loads the reference script would reject (a state dict that does
# not fit its model) into working ones, and leave every load it accepts unchanged
_EXTRA_KEYS = {"ffn_dim": None, "pope_fused": False}


def config_from_checkpoint(checkpoint: dict) -> TransformerConfig:
    """The TransformerConfig the reference script builds: ``config["model"]`` if present, else
    ``model_config``.  Keys it does not read (norm_eps, use_qk_norm, tie_embeddings) keep their
    defaults, as there."""
    cfg = checkpoint.get("config", {}) or {}
    model_cfg = cfg.get("model", checkpoint.get("model_config", {})) if isinstance(cfg, dict) else {}
    model_cfg = model_cfg or {}
    keys = dict(_CONFIG_KEYS, **_EXTRA_KEYS)
    return TransformerConfig(**{k: model_cfg.get(k, d) for k, d in keys.items()})


def load_model(checkpoint_path: str, device: torch.device) -> tuple[Transformer, TransformerConfig, str]:
    """(model on ``device`` in eval mode, its config, pe_mode) from a trainer checkpoint; strips a
    ``torch.compile`` ``_orig_mod.`` prefix from the state-dict keys and loads strictly."""
    checkpoint = torch.load(checkpoint_path, map_location="cpu", weights_only=True)
    config = config_from_checkpoint(checkpoint)
    model = Transformer(config)
    state = checkpoint["model_state_dict"]
    if any(k.startswith("_orig_mod.") for k in state):
        state = {k.replace("_orig_mod.", ""): v for k, v in state.items()}
    model.load_state_dict(state)
    return model.to(device).eval(), config, config.pe_mode


def save_checkpoint(model: Transformer, path: str, step: int = 0) -> None:
    """Write ``model`` in the reference trainer's checkpoint layout (the keys load_model reads,
    plus step / tokens_seen / epoch), for round trips and for handing weights to the reference."""
    torch.save({
        "model_state_dict": model.state_dict(),
        "step": step,
        "tokens_seen": 0,
        "epoch": 0,
        "config": {},
        "model_config": dict(model.config.__dict__),
    }, path)


def clear_memory() -> None:
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
        torch.cuda.synchronize()


@torch.inference_mode()
def compute_ppl_sliding_window(model, tokens: Sequence[int], context_length: int, device: torch.device,
                               stride: Optional[int] = None, dtype: Optional[torch.dtype] = None
                               ) -> tuple[float, bool]:
    """(perplexity, oom) over sliding windows (scripts/evaluate_long_context.py:80-137).

    ``dtype`` (an addition): run the forward under autocast to this dtype; None = the model's own
    precision, as the reference."""
    model.extend_context_length(context_length)
    if stride is None:
        stride = context_length // 2
    total_loss = 0.0
    total_tokens = 0
    oom = False
    tokens = list(tokens[:min(len(tokens), context_length * 4)])
    for start in range(0, len(tokens) - context_length, stride):
        chunk = tokens[start:start + context_length]
        input_ids = torch.tensor([chunk], device=device)
        try:
            if dtype is not None and dtype != torch.float32:
                with torch.autocast(device_type=torch.device(device).type, dtype=dtype):
                    loss = model(input_ids, labels=input_ids)["loss"].item()
            else:
                loss = model(input_ids, labels=input_ids)["loss"].item()
            n_tokens = context_length // 2
            total_loss += loss * n_tokens
            total_tokens += n_tokens
            if total_tokens >= context_length * 2:
                break
        except RuntimeError as e:
            if "out of memory" in str(e).lower():
                oom = True
                clear_memory()
                break
            raise
        clear_memory()
    if total_tokens == 0:
        return float("inf"), oom
    avg = total_loss / total_tokens
    return (math.exp(avg) if avg < 20 else float("inf")), oom


def load_tokens(path: str) -> list[int]:
    """Token ids from ``.npy`` (integer array, loaded without pickle) or whitespace-separated text."""
    if path.endswith(".npy"):
        import numpy as np
        return [int(t) for t in np.load(path, allow_pickle=False).reshape(-1)]
    with open(path) as f:
        return [int(t) for t in f.read().split()]


def _status(ratio: float, first: bool) -> str:
    if first:
        return "baseline"
    return ("excellent" if ratio < 1.2 else "good" if ratio < 1.5 else "degraded" if ratio < 2.0
            else "poor" if ratio < 5.0 else "BROKEN")


def evaluate(checkpoint_dir: str, tokens: list[int], context_lengths: list[int], device: torch.device,
             models: Optional[list[str]] = None, dtype: Optional[torch.dtype] = None) -> dict:
    """Per model directory (latest checkpoint_step_*.pt), PPL and ratio to the first length
    (scripts/evaluate_long_context.py:177-225)."""
    model_dirs = sorted(d for d in Path(checkpoint_dir).iterdir() if d.is_dir())
    if models:
        model_dirs = [d for d in model_dirs if d.name in models]
    results = {}
    for model_dir in model_dirs:
        ckpts = sorted(model_dir.glob("checkpoint_step_*.pt"))
        if not ckpts:
            continue
        model, config, pe_mode = load_model(str(ckpts[-1]), device)
        print(f"\n{model_dir.name}:\n  PE mode: {pe_mode}, params: {config.num_params:,}", flush=True)
        res = {"ppl": {}, "ratio": {}, "pe_mode": pe_mode}
        base = None
        for i, ctx in enumerate(context_lengths):
            ppl, oom = compute_ppl_sliding_window(model, tokens, ctx, device, dtype=dtype)
            if oom:
                print(f"  {ctx:>6}: OOM", flush=True)
                break
            res["ppl"][ctx] = ppl
            base = ppl if base is None else base
            ratio = ppl / base if base > 0 else float("inf")
            res["ratio"][ctx] = ratio
            print(f"  {ctx:>6}: PPL={ppl:>8.1f}, ratio={ratio:.2f}x [{_status(ratio, i == 0)}]", flush=True)
        results[model_dir.name] = res
        del model
        clear_memory()
    return results


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Long context PPL evaluation (fused HIP attention)")
    ap.add_argument("--checkpoint-dir", default="checkpoints/1b")
    ap.add_argument("--output-dir", default="eval_results/long_context")
    ap.add_argument("--context-lengths", type=int, nargs="+",
                    default=[512, 1024, 2048, 4096, 8192, 16384, 32768])
    ap.add_argument("--device", default="cuda:0")
    ap.add_argument("--models", nargs="+", default=None)
    ap.add_argument("--tokens", required=True, help=".npy of token ids or a text file of whitespace-separated ids")
    ap.add_argument("--dtype", choices=["fp32", "bf16"], default="fp32")
    args = ap.parse_args(argv)
    device = torch.device(args.device)
    out_dir = Path(args.output_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    tokens = load_tokens(args.tokens)
    print(f"Loaded {len(tokens):,} tokens", flush=True)
    results = evaluate(args.checkpoint_dir, tokens, args.context_lengths, device, args.models,
                       torch.bfloat16 if args.dtype == "bf16" else None)

    def last_ratio(name):
        r = list(results[name]["ratio"].values())
        return r[-1] if r else 999

    print("\n" + "=" * 80 + "\nSUMMARY: PPL Degradation Ratio (lower is better)\n" + "=" * 80)
    print(f"{'Model':<20}" + "".join(f" | {c:>7}" for c in args.context_lengths))
    for name in sorted(results, key=last_ratio):
        cells = []
        for c in args.context_lengths:
            r = results[name]["ratio"].get(c, float("nan"))
            cells.append(f" | {'OOM':>7}" if math.isnan(r) else
                         f" | {r:>6.2f}{'' if r < 1.5 else '*' if r < 3 else '**'}")
        print(f"{name:<20}" + "".join(cells))
    out_file = out_dir / "long_context_ppl.json"
    with open(out_file, "w") as f:
        json.dump({n: {"pe_mode": r["pe_mode"], "ppl": {str(k): v for k, v in r["ppl"].items()},
                       "ratio": {str(k): v for k, v in r["ratio"].items()}} for n, r in results.items()},
                  f, indent=2)
    print(f"\nResults saved to {out_file}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
