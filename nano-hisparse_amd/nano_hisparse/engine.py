"""Round-robin decode scheduler with host, index and device admission.

Reference: nano_hisparse/engine.py:12-143. Each step admits at most one
waiting prompt (prefill) and gives every running request one greedy decode
turn; requests are released when they finish or are cancelled.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from .config import CapacityError
from .model import Model


@dataclass
class Request:
    request_id: str
    prompt: list
    max_new_tokens: int
    generated: list = field(default_factory=list)
    prefill_count: int = 0
    decode_count: int = 0
    finished: bool = False
    cancelled: bool = False


class Engine:
    def __init__(self, model: Model, cache, top_k=None, backend="auto", eos_token_id=None, selector="quest",
                 batch_decode=False, micro_batches=1, graph=False):
        """batch_decode=True gives all running requests their decode turn in
        one Model.decode_batch call (GPU cache, Quest top_k; micro_batches=2
        pipelines two halves of the batch; graph=True replays each batch
        composition's step from a captured HIP graph); emission order and
        admission are unchanged."""
        cfg, kv = model.config, cache.config
        if (cfg.num_key_value_heads, cfg.head_dim) != (kv.kv_heads, kv.head_dim):
            raise ValueError("model/cache head dimensions differ")
        if model.device != cache.pool.device or model.dtype != cache.pool.dtype:
            raise ValueError("model/cache dtype or device differ")
        if top_k is not None and top_k < 1:
            raise ValueError("top_k must be positive or None")
        self.model, self.cache, self.top_k, self.backend = model, cache, top_k, backend
        self.eos_token_id = eos_token_id
        self.selector = selector
        if batch_decode and (top_k is None or selector != "quest" or not cache.storage.cuda):
            raise ValueError("batched decode needs a GPU cache and the Quest selector with a top_k")
        self.batch_decode = batch_decode
        self.micro_batches = micro_batches
        self.graph = graph
        if graph and not batch_decode:
            raise ValueError("graph replay needs batch_decode")
        self.requests: dict = {}
        self.waiting: deque = deque()
        self.running: deque = deque()

    def add_request(self, request_id, prompt, max_new_tokens=16):
        if request_id in self.requests or not prompt or max_new_tokens < 1:
            raise ValueError("need a unique ID, nonempty prompt, and positive output length")
        if any(t < 0 or t >= self.model.config.vocab_size for t in prompt):
            raise ValueError("token outside model vocabulary")
        layers = self.model.config.num_hidden_layers
        total = len(prompt) + max_new_tokens
        pages = -(-total // self.cache.config.page_size)
        if pages * layers > self.cache.config.host_pages:
            raise CapacityError("request cannot fit even in an empty host pool")
        if self.cache.admission_blocks(layers) > self.cache.budget:
            raise CapacityError("request hot-region + tail footprint cannot fit the device pool")
        if self.cache.index_reservation_bytes(total, layers) > self.cache.config.index_budget_bytes:
            raise CapacityError("request index cannot fit even in an empty index budget")
        request = Request(request_id, list(prompt), max_new_tokens)
        self.requests[request_id] = request
        self.waiting.append(request)
        return request

    def _emit(self, request, logits=None, token=None):
        if token is None:
            token = int(logits.argmax().item())
        request.generated.append(token)
        if token == self.eos_token_id or len(request.generated) >= request.max_new_tokens:
            request.finished = True
            self.cache.release_request(request.request_id, wait=False)
        return token

    def _admit(self, request):
        layers = self.model.config.num_hidden_layers
        total = len(request.prompt) + request.max_new_tokens
        try:
            self.cache.reserve(request.request_id, total, layers)
            return True
        except CapacityError:
            if self.running:
                return False  # retry after running requests progress
            if not self.cache.storage.retired:
                raise
            self.cache.collect(wait=True)  # idle: wait for retirements
            self.cache.reserve(request.request_id, total, layers)
            return True

    def step(self):
        """Admit at most one prompt, then one decode turn per running request.

        Returns [(request_id, token)] in emission order.
        """
        emitted = []
        self.cache.collect()
        if self.waiting and self._admit(self.waiting[0]):
            request = self.waiting.popleft()
            logits = self.model.prefill(request.prompt, self.cache, request.request_id)
            request.prefill_count += 1
            emitted.append((request.request_id, self._emit(request, logits)))
            if not request.finished:
                self.running.append(request)
        if self.batch_decode and self.running:
            batch = list(self.running)
            self.running.clear()
            logits = self.model.decode_batch(
                [r.generated[-1] for r in batch], [r.request_id for r in batch], self.cache, self.top_k,
                micro_batches=self.micro_batches, graph=self.graph,
            )
            for request, token in zip(batch, logits.argmax(-1).tolist()):
                request.decode_count += 1
                emitted.append((request.request_id, self._emit(request, token=token)))
                if not request.finished:
                    self.running.append(request)
            return emitted
        for _ in range(len(self.running)):
            request = self.running.popleft()
            logits = self.model.decode(
                request.generated[-1], request.request_id, self.cache, self.top_k, self.backend,
                selector=self.selector,
            )
            request.decode_count += 1
            emitted.append((request.request_id, self._emit(request, logits)))
            if not request.finished:
                self.running.append(request)
        return emitted

    def run(self):
        while self.waiting or self.running:
            self.step()
        self.cache.collect(wait=True)
        return {name: request.generated for name, request in self.requests.items()}

    def cancel(self, request_id):
        request = self.requests[request_id]
        if request.finished:
            return
        if request in self.waiting:
            self.waiting.remove(request)
        else:
            self.running.remove(request)
            self.cache.release_request(request_id, wait=False)
        request.finished = request.cancelled = True
