"""Writes reference_plumbing_tokens.json: the greedy token streams and row
counters of the CPU plumbing config, produced by the reference package
itself (imported from /root/reference, run on the CPU through its torch
path), so the engine's end-to-end output is pinned against the reference and
not only against the oracle.

The config is the one tests/test_workloads.py runs (run_plumbing_config): a
random-init 2-layer decoder (hidden 256, 4/2 heads of 64, MLP 688, vocab
32000, fp32, torch seed 42, reference model.py:75-96 construction order), 3
prompts of 512 tokens from a torch Generator seeded 42, pages of 16, Quest
top-8 pages, hot rows 128, a pool of 3x one hot region + 2 tails per layer,
64 greedy tokens each, round robin (reference engine.py:76-126). One torch
thread, as the reference CLI sets (cli.py:67).

Run from the repository root in this container (the reference is not on the
GPU host): python tests/golden/make_reference_tokens.py
"""

import json
import os
import sys

REFERENCE = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_plumbing_tokens.json")


def main():
    # the reference tree is read-only: importing it must not write bytecode there
    sys.dont_write_bytecode = True
    # the reference's package, not this repository's (same package name)
    sys.path[:] = [REFERENCE] + [p for p in sys.path if "nano-hisparse_amd" not in p and p not in ("", ".")]
    import torch

    import nano_hisparse
    from nano_hisparse.config import CacheConfig
    from nano_hisparse.engine import Engine
    from nano_hisparse.hybrid import HotConfig, HybridKVCache
    from nano_hisparse.model import Model, ModelConfig

    assert os.path.realpath(nano_hisparse.__file__).startswith(REFERENCE), nano_hisparse.__file__
    torch.set_num_threads(1)
    torch.manual_seed(42)
    cfg = ModelConfig(vocab_size=32000, hidden_size=256, intermediate_size=688, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    model = Model(cfg).eval()
    P, top, T, new = 16, 8, 512, 64
    hot = HotConfig(top * P, top * P)
    g = torch.Generator().manual_seed(42)
    prompts = [torch.randint(0, cfg.vocab_size, (T,), generator=g).tolist() for _ in range(3)]
    kv = CacheConfig(gpu_pages=3 * hot.admission_blocks(P, cfg.num_hidden_layers),
                     host_pages=3 * cfg.num_hidden_layers * -(-(T + new) // P), page_size=P, kv_heads=2,
                     head_dim=64, device="cpu")
    cache = HybridKVCache(kv, hot)
    engine = Engine(model, cache, top_k=top)
    for i, prompt in enumerate(prompts):
        engine.add_request(f"p{i}", prompt, new)
    out = engine.run()
    cache.assert_invariants()
    stats = cache.snapshot()["row_stats"]
    record = {
        "source": "reference package (nano_hisparse, imported from /root/reference) on the CPU, torch "
                  + torch.__version__ + ", 1 thread",
        "config": {"layers": 2, "hidden": 256, "heads": [4, 2], "mlp": 688, "vocab": 32000, "seed": 42,
                   "prompts": 3, "prompt_tokens": T, "page_size": P, "top_pages": top, "hot_rows": top * P,
                   "new_tokens": new},
        "tokens": {k: [int(t) for t in v] for k, v in sorted(out.items())},
        "row_stats": {k: int(v) for k, v in stats.items()},
    }
    with open(OUT, "w") as f:
        json.dump(record, f, indent=1)
        f.write("\n")
    print("wrote", OUT, {k: len(v) for k, v in record["tokens"].items()}, record["row_stats"])


if __name__ == "__main__":
    main()
