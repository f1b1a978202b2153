"""Writes a small expert cache in the reference's on-disk format, as
tinygiant/relayout.py:147-162 (layer files) and :287-300 (index.json) lay it
out: per layer, every expert's gate, up and down bytes back to back in
expert-id order, and an index with each expert's offset and sizes."""

import json
from pathlib import Path

import numpy as np

KEYS = ("gate", "up", "down")
NAMES = {0: "q4_k", 1: "float16", 2: "q6_k", 3: "mxfp4", 4: "q8_0"}


def write_cache(cache_dir, layers, n_experts, embed_dim, inter_dim, formats, omit_formats=()):
    """layers: {layer: {expert_id: {key: uint8 array}}}; formats: {key: code}.
    Layers listed in omit_formats get no tensor_formats entry (a reader then
    assumes q4_k).  Returns the index dict."""
    d = Path(cache_dir)
    d.mkdir(parents=True, exist_ok=True)
    index = {"magic": "NWSMOE01", "version": 2, "n_layers": len(layers), "n_experts": n_experts,
             "embed_dim": embed_dim, "dtype": "quant",
             "q4_sizes": {"gate": {"out_dim": inter_dim, "in_dim": embed_dim},
                          "up": {"out_dim": inter_dim, "in_dim": embed_dim},
                          "down": {"out_dim": embed_dim, "in_dim": inter_dim}},
             "layers": {}}
    for layer, experts in layers.items():
        name = f"layer_{layer:03d}.q4.bin"
        offsets, cur = {}, 0
        with open(d / name, "wb") as f:
            for eid in sorted(experts):
                sizes = {}
                start = cur
                for k in KEYS:
                    b = np.ascontiguousarray(experts[eid][k], np.uint8)
                    f.write(b.tobytes())
                    sizes[k] = int(b.nbytes)
                    cur += b.nbytes
                offsets[str(eid)] = {"offset": start, "sizes": sizes}
        entry = {"file": name, "total_bytes": cur, "expert_offsets": offsets}
        if layer not in omit_formats:
            entry["tensor_formats"] = {k: NAMES[formats[k]] for k in KEYS}
        index["layers"][str(layer)] = entry
    with open(d / "index.json", "w") as f:
        json.dump(index, f, indent=2)
    return index


def synth_layers(n_layers, n_experts, embed_dim, inter_dim, formats, seed):
    import tinygiant_amd.synth as S
    out = {}
    for layer in range(n_layers):
        out[layer] = {}
        for e in range(n_experts):
            out[layer][e] = {
                "gate": S.matrix_host(formats["gate"], S.tensor_seed(seed, layer, e, 0), inter_dim, embed_dim),
                "up": S.matrix_host(formats["up"], S.tensor_seed(seed, layer, e, 1), inter_dim, embed_dim),
                "down": S.matrix_host(formats["down"], S.tensor_seed(seed, layer, e, 2), embed_dim, inter_dim),
            }
    return out
