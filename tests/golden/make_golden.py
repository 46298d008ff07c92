"""Write the golden fixtures under tests/golden/ from the reference's Decision/ data.

Run once in the build container (the reference tree is not present on the GPU
box; the fixtures it writes are committed):

    python tests/golden/make_golden.py [/root/reference]

Outputs (data only -- inputs and expected outputs; no reference code):

* ``decision_topk_kat.npz`` -- for a fixed selection of layers of three
  released maps: the per-tile score matrix (input) and the released BF16 tile
  ids for keep01/keep05/keep20 (expected output of the top-k mask rule,
  src/quantization/decisions.py:174-183).  Keys ``<set>__<stem>__scores``,
  ``<set>__<stem>__keepXX``.
* ``llama32_3b_gi_keep01/fp16_keep_ids_tile64x64.npz`` and
  ``llama32_3b_gi_keep05/...`` -- two released tile-map archives byte-for-byte
  (format fixture for mask_io and the real Llama-3.2-3B masks used by the
  end-to-end path).
"""
from __future__ import annotations

import shutil
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

# (label, model folder, style, stems) -- stems chosen to cover every projection
# shape of each model (square, narrow K/V, wide MLP, transposed down).
SELECTION = [
    ("llama_iaa", "meta-llama_Llama-3.2-3B-Instruct", "iaa",
     ["model_layers_0_self_attn_q_proj", "model_layers_0_self_attn_k_proj",
      "model_layers_5_mlp_gate_proj", "model_layers_27_mlp_down_proj"]),
    ("qwen7b_gi", "Qwen_Qwen2.5-7B-Instruct", "gi",
     ["model_layers_3_self_attn_v_proj", "model_layers_10_mlp_up_proj", "model_layers_20_self_attn_o_proj"]),
    ("qwen14b_iaa", "Qwen_Qwen2.5-14B-Instruct", "iaa",
     ["model_layers_1_self_attn_k_proj", "model_layers_40_mlp_down_proj"]),
]
KEEPS = ("keep01", "keep05", "keep20")


def main(ref_root: str = "/root/reference") -> None:
    dec = Path(ref_root) / "Decision"
    out = {}
    for label, model, style, stems in SELECTION:
        base = dec / model / style
        with np.load(base / f"{style}_tile_scores_tile64x64.npz", allow_pickle=False) as scores:
            for stem in stems:
                out[f"{label}__{stem}__scores"] = np.asarray(scores[stem], dtype=np.float32)
        for keep in KEEPS:
            with np.load(base / "tile_masks" / keep / "fp16_keep_ids_tile64x64.npz", allow_pickle=False) as d:
                names = [str(s) for s in d["stems"].tolist()]
                for stem in stems:
                    i = names.index(stem)
                    out[f"{label}__{stem}__{keep}"] = np.asarray(d[f"ids_{i}"])
                    out[f"{label}__{stem}__shape"] = np.asarray(d[f"shape_{i}"])
    np.savez_compressed(HERE / "decision_topk_kat.npz", **out)
    for keep in ("keep01", "keep05"):
        src = dec / "meta-llama_Llama-3.2-3B-Instruct" / "gi" / "tile_masks" / keep / "fp16_keep_ids_tile64x64.npz"
        dst = HERE / f"llama32_3b_gi_{keep}" / "fp16_keep_ids_tile64x64.npz"
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(src, dst)
    print("wrote", sorted(p.name for p in HERE.iterdir()))


if __name__ == "__main__":
    main(*sys.argv[1:])
