"""The decoder and the engine over the hybrid cache: sparse decode through
the cache matches dense generation, admission back-pressure, cancellation
and the Hugging Face Qwen2 weight layout.

Scenarios follow the reference's tests/test_engine.py:10-103 and
tests/test_model.py:8-95.
"""

import pytest
import torch

from nano_hisparse.config import CacheConfig, CapacityError
from nano_hisparse.engine import Engine
from nano_hisparse.hybrid import HotConfig, HybridKVCache
from nano_hisparse.model import Model, ModelConfig

TINY = dict(hidden_size=32, intermediate_size=64, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, vocab_size=64)


def tiny_model(device="cpu"):
    return Model(ModelConfig(**TINY)).eval().to(device)


def cache_for(device, gpu_pages, hot, host_pages=64, page_size=4):
    cfg = CacheConfig(gpu_pages=gpu_pages, host_pages=host_pages, page_size=page_size, kv_heads=2, head_dim=8,
                      device=device)
    return HybridKVCache(cfg, hot)


@pytest.mark.parametrize("top_k", [None, 2])
def test_offloaded_generation_matches_fully_resident_generation(device, top_k):
    torch.manual_seed(31)
    model = tiny_model(device)
    union = 28 if top_k is None else 8
    hot = HotConfig(union, union)
    prompts = {"a": list(range(1, 18)), "b": list(range(8, 30))}
    results = []
    for budget in (64, hot.admission_blocks(4, 2)):
        cache = cache_for(device, budget, hot)
        engine = Engine(model, cache, top_k=top_k)
        engine.add_request("a", prompts["a"], 8)
        engine.add_request("b", prompts["b"], 6)
        engine.step()
        if budget != 64:
            assert len(engine.waiting) == 1  # "b" waits for device credits
        results.append(engine.run())
        assert all(r.prefill_count == 1 for r in engine.requests.values())
        assert all(r.decode_count == r.max_new_tokens - 1 for r in engine.requests.values())
        assert not cache.storage.requests and not cache.tables and not any(cache.owners)
        if budget != 64:
            assert cache.snapshot()["row_stats"]["misses"] > 0
        cache.assert_invariants()
    assert results[0] == results[1]
    if top_k is None:  # dense decoding reproduces the full causal forward
        for name, prompt in prompts.items():
            history = list(prompt)
            for token in results[0][name]:
                assert model.prefill(history).argmax().item() == token
                history.append(token)


def test_host_back_pressure_admits_waiters_eventually(cpu_kernels):
    torch.manual_seed(4)
    model = tiny_model()
    cache = cache_for("cpu", 24, HotConfig(16, 16), host_pages=8)
    engine = Engine(model, cache)
    for i in range(3):
        engine.add_request(str(i), [1] * 10, 5)
    engine.step()
    assert len(engine.waiting) == 2
    engine.run()
    assert all(len(r.generated) == 5 and r.prefill_count == 1 for r in engine.requests.values())


def test_cancelling_requests_returns_all_capacity(cpu_kernels):
    model = tiny_model()
    cache = cache_for("cpu", 8, HotConfig(8, 8))
    engine = Engine(model, cache, top_k=2)
    for name in ("a", "b", "c"):
        engine.add_request(name, list(range(1, 22)), 5)
    engine.step()
    engine.cancel("a")
    engine.cancel("b")
    outputs = engine.run()
    assert len(outputs["c"]) == 5
    assert engine.requests["a"].cancelled and engine.requests["b"].prefill_count == 0
    assert not any(cache.owners) and len(cache.storage.free_host) == 64
    cache.assert_invariants()
    with pytest.raises(CapacityError, match="host"):
        engine.add_request("too-long", [1] * 1000, 2)


def test_engine_rejects_bad_requests(cpu_kernels):
    engine = Engine(tiny_model(), cache_for("cpu", 16, HotConfig(8, 8)))
    engine.add_request("a", [1, 2], 2)
    for args in (("a", [1], 1), ("b", [], 1), ("c", [1], 0)):
        with pytest.raises(ValueError, match="unique"):
            engine.add_request(*args)
    with pytest.raises(ValueError, match="vocabulary"):
        engine.add_request("d", [64], 1)


def test_decode_through_offloaded_cache_matches_full_forward(device):
    torch.manual_seed(31)
    model = tiny_model(device)
    hot = HotConfig(24, 24)
    cache = cache_for(device, hot.admission_blocks(4, 2), hot)
    history = list(range(1, 18))
    cache.reserve("a", 24, 2)
    torch.testing.assert_close(model.prefill(history, cache, "a"), model.prefill(history))
    cache.storage.synchronize()
    for layer in range(2):
        cache.reclaim_history("a", layer, evict=True)
    for token in (18, 19, 20):
        history.append(token)
        torch.testing.assert_close(model.decode(token, "a", cache), model.prefill(history), atol=3e-6, rtol=3e-5)
    assert cache.snapshot()["row_stats"]["misses"] > 0
    with pytest.raises(ValueError, match="exactly once"):
        model.prefill(history, cache, "a")
    cache.release_request("a")
    cache.assert_invariants()


def test_qwen2_weights_and_logits_match_transformers(cpu_kernels, tmp_path):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(8)
    cfg = ModelConfig(**TINY)
    hf_cfg = transformers.Qwen2Config(**vars(cfg), attention_dropout=0, tie_word_embeddings=False)
    hf = transformers.Qwen2ForCausalLM(hf_cfg).eval()
    model = Model(cfg).eval()
    model.load_state_dict(hf.state_dict(), strict=True)
    hf.save_pretrained(tmp_path)
    loaded = Model.from_pretrained(str(tmp_path), device="cpu", dtype=torch.float32)
    tokens = [1, 7, 3, 4, 9, 11, 17]
    with torch.inference_mode():
        expected = hf(torch.tensor([tokens])).logits[0, -1]
    torch.testing.assert_close(model.prefill(tokens), expected, atol=2e-6, rtol=2e-5)
    torch.testing.assert_close(loaded.prefill(tokens), expected, atol=2e-6, rtol=2e-5)
    cache = HybridKVCache(
        CacheConfig(gpu_pages=12, host_pages=16, page_size=3, kv_heads=2, head_dim=8, device="cpu"), HotConfig(12, 12)
    )
    cache.reserve("a", 12, 2)
    model.prefill(tokens, cache, "a")
    for token in (12, 19, 5):
        tokens.append(token)
        with torch.inference_mode():
            expected = hf(torch.tensor([tokens])).logits[0, -1]
        torch.testing.assert_close(model.decode(token, "a", cache), expected, atol=2e-6, rtol=2e-5)
    cache.release_request("a")
    cache.assert_invariants()
