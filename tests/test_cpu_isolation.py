"""A CPU cache never loads libnhs_hip.so (reference tests/test_cli.py:9-41:
the CPU path must not touch the GPU extension). A fresh interpreter runs a
CPU engine end to end with the oracle as the CPU kernel provider and then
checks its own memory map; without a provider the CPU path refuses to run."""

import os
import subprocess
import sys
import textwrap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = textwrap.dedent(
    """
    import sys
    sys.path[:0] = [{root!r}, {pkg!r}, {tests!r}]
    import torch
    import cpu_provider
    from nano_hisparse import _hip
    from nano_hisparse.config import CacheConfig
    from nano_hisparse.engine import Engine
    from nano_hisparse.hybrid import HotConfig, HybridKVCache
    from nano_hisparse.model import Model, ModelConfig

    torch.manual_seed(0)
    model = Model(ModelConfig(hidden_size=32, intermediate_size=64, num_hidden_layers=2, num_attention_heads=4,
                              num_key_value_heads=2, vocab_size=64)).eval()
    cfg = CacheConfig(gpu_pages=16, host_pages=64, page_size=4, kv_heads=2, head_dim=8, device="cpu")
    try:
        engine = Engine(model, HybridKVCache(cfg, HotConfig(8, 8)), top_k=2)
        engine.add_request("x", list(range(1, 20)), 3)
        engine.run()
        raise SystemExit("the CPU path ran without a kernel provider")
    except RuntimeError as exc:
        assert "provider" in str(exc), exc
    cpu_provider.install()
    engine = Engine(model, HybridKVCache(cfg, HotConfig(8, 8)), top_k=2)
    engine.add_request("a", list(range(1, 20)), 4)
    out = engine.run()
    assert len(out["a"]) == 4
    maps = open("/proc/self/maps").read()
    assert "libnhs_hip" not in maps and _hip._lib is None, "libnhs_hip.so was loaded"
    print("ok")
    """
)


def test_cpu_engine_never_loads_the_hip_library():
    code = SCRIPT.format(root=ROOT, pkg=os.path.join(ROOT, "nano-hisparse_amd"), tests=os.path.join(ROOT, "tests"))
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
    result = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300, env=env)
    assert result.returncode == 0 and result.stdout.strip().endswith("ok"), result.stdout + result.stderr
