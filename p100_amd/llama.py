"""Greedy decode of a Llama-architecture model through libp1x's decode step (p1x_llama_decode_step).

The 8B shape is the one the reference's decode ceiling models (bin/decode-model.py:52-57: 32 layers, hidden 4096,
FFN 14336, 32/8 heads of 128, vocab 128256) and its llama-bench decode runs measure (bench/phase0.sh:124). Weights
are random-init (there are no checkpoints here): N(0, std) quantized with the ggml reference rules of
``p100_amd.synth``, norm weights 1 + N(0, 0.1), fp16 KV caches.

Every position-dependent quantity of a step lives in device memory (``state``: pos, n_prompt, n_kv), so
``Decoder.capture()`` records one step into a HIP graph and ``Decoder.run()`` replays it once per position:
prompt positions take their token from ``prompt``, later ones the model's own argmax from ``tokens``.
"""
from __future__ import annotations

import ctypes as C

from . import Q4_0, _check, _ptr, _stream, load, row_bytes
from . import synth

vp = C.c_void_p


class LlamaHParams(C.Structure):
    """p1x_llama_hparams."""

    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "n_ff", "n_vocab", "n_ctx",
                                      "wtype", "embd_type", "output_type")] + [
        ("rms_eps", C.c_float), ("rope_base", C.c_float)]

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head


class LlamaLayer(C.Structure):
    """p1x_llama_layer."""

    _fields_ = [(n, vp) for n in ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up", "w_down",
                                  "k_cache", "v_cache")]


class LlamaModelC(C.Structure):
    """p1x_llama_model."""

    _fields_ = [("hp", LlamaHParams), ("tok_embd", vp), ("layers", C.POINTER(LlamaLayer)), ("output_norm", vp),
                ("output", vp)]


LLAMA3_8B = dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, n_ff=14336, n_vocab=128256)


def hparams(n_ctx: int, wtype=Q4_0, embd_type=Q4_0, output_type=None, rms_eps=1e-5, rope_base=500000.0,
            **dims) -> LlamaHParams:
    """Hyper-parameters; dims default to the Llama-3-8B shape."""
    d = dict(LLAMA3_8B)
    d.update(dims)
    return LlamaHParams(d["n_layer"], d["n_embd"], d["n_head"], d["n_head_kv"], d["n_ff"], d["n_vocab"], n_ctx, wtype,
                        embd_type, wtype if output_type is None else output_type, rms_eps, rope_base)


class LlamaModel:
    """Random-init weights and KV caches on `device`. q/k/v rows and gate/up rows are allocated back to back, so
    the step runs each group as one mat-vec launch."""

    def __init__(self, hp: LlamaHParams, device="cuda", seed=0, std=0.02):
        import torch

        self.hp = hp
        E, F, d = hp.n_embd, hp.n_ff, hp.head_dim
        kv = hp.n_head_kv * d
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)

        def weights(t, rows, k):
            return synth.random_weights(t, rows, k, std=std, generator=gen, device=device)

        def norm():
            return 1.0 + 0.1 * torch.randn(E, generator=gen, device=device)

        self.tok_embd = weights(hp.embd_type, hp.n_vocab, E)
        self.layers = []
        for _ in range(hp.n_layer):
            self.layers.append(dict(
                attn_norm=norm(), wqkv=weights(hp.wtype, E + 2 * kv, E), wo=weights(hp.wtype, E, E),
                ffn_norm=norm(), w_gate_up=weights(hp.wtype, 2 * F, E), w_down=weights(hp.wtype, E, F),
                k_cache=torch.zeros((hp.n_head_kv, hp.n_ctx, d), dtype=torch.float16, device=device),
                v_cache=torch.zeros((hp.n_head_kv, hp.n_ctx, d), dtype=torch.float16, device=device)))
        self.output_norm = norm()
        self.output = weights(hp.output_type, hp.n_vocab, E)
        self._c = self._c_struct()

    def _c_struct(self) -> LlamaModelC:
        hp = self.hp
        E, F, kv = hp.n_embd, hp.n_ff, hp.n_head_kv * hp.head_dim
        nb = row_bytes(hp.wtype, E)
        arr = (LlamaLayer * hp.n_layer)()
        for i, L in enumerate(self.layers):
            q = L["wqkv"].data_ptr()
            g = L["w_gate_up"].data_ptr()
            arr[i] = LlamaLayer(L["attn_norm"].data_ptr(), q, q + E * nb, q + (E + kv) * nb, L["wo"].data_ptr(),
                                L["ffn_norm"].data_ptr(), g, g + F * nb, L["w_down"].data_ptr(),
                                L["k_cache"].data_ptr(), L["v_cache"].data_ptr())
        self._layers_c = arr  # kept alive: the struct points at it
        return LlamaModelC(hp, self.tok_embd.data_ptr(), arr, self.output_norm.data_ptr(), self.output.data_ptr())

    def weight_bytes(self) -> int:
        """Bytes of every matrix a decode step reads (the layers and the output projection; the embedding reads one
        row)."""
        hp = self.hp
        per_layer = sum(self.layers[0][k].numel() for k in ("wqkv", "wo", "w_gate_up", "w_down"))
        return hp.n_layer * per_layer + self.output.numel()

    def layer_tensors(self, i):
        """Views of layer i: wq, wk, wv, w_gate, w_up row blocks (uint8 [rows, row_bytes])."""
        hp = self.hp
        E, F, kv = hp.n_embd, hp.n_ff, hp.n_head_kv * hp.head_dim
        L = self.layers[i]
        return dict(wq=L["wqkv"][:E], wk=L["wqkv"][E:E + kv], wv=L["wqkv"][E + kv:], w_gate=L["w_gate_up"][:F],
                    w_up=L["w_gate_up"][F:])


class Decoder:
    """Device-resident greedy decode over a LlamaModel."""

    def __init__(self, model: LlamaModel, max_prompt: int):
        import torch

        self.model = model
        hp = model.hp
        dev = model.output.device
        self.lib = load()
        self.state = torch.zeros(4, dtype=torch.int32, device=dev)  # p1x_decode_state
        self.prompt = torch.zeros(max(max_prompt, 1), dtype=torch.int32, device=dev)
        self.tokens = torch.zeros(hp.n_ctx + 1, dtype=torch.int32, device=dev)
        self.logits = torch.empty(hp.n_vocab, dtype=torch.float32, device=dev)
        need = self.lib.p1x_llama_workspace(C.byref(hp))
        if need == 0:
            raise ValueError("invalid hyper-parameters")
        self.ws = torch.empty(need, dtype=torch.uint8, device=dev)
        self.graph = None

    def reset(self, prompt_ids):
        """Positions restart at 0 with this prompt (host sequence of token ids); the caches are overwritten as the
        positions are decoded again."""
        import torch

        n = len(prompt_ids)
        if n > self.prompt.numel() or n > self.model.hp.n_ctx:
            raise ValueError("prompt longer than the decoder's capacity")
        if n:
            self.prompt[:n].copy_(torch.as_tensor(list(prompt_ids), dtype=torch.int32))
        self.state.copy_(torch.tensor([0, n, 0, 0], dtype=torch.int32))
        self.tokens.zero_()

    def step(self, stream=None):
        """Enqueues one decode step (one position)."""
        _check(self.lib.p1x_llama_decode_step(C.byref(self.model._c), _ptr(self.state), _ptr(self.prompt),
                                              _ptr(self.tokens), _ptr(self.logits), _ptr(self.ws), self.ws.numel(),
                                              _stream(stream)))

    def capture(self):
        """Records one step into a graph (the state is left as it was)."""
        import torch

        saved = self.state.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step(s)  # warm-up on the side stream, as graph capture expects
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        torch.cuda.synchronize()
        self.state.copy_(saved)
        self.graph = g
        return g

    def run(self, n_steps: int, use_graph=True):
        """Decodes n_steps positions from the current state."""
        if use_graph and self.graph is None:
            self.capture()
        for _ in range(n_steps):
            if use_graph:
                self.graph.replay()
            else:
                self.step()

    def generate(self, prompt_ids, n_gen: int, use_graph=True):
        """Greedy continuation: the n_gen tokens predicted after the prompt (host list)."""
        import torch

        n = len(prompt_ids)
        self.reset(prompt_ids)
        self.run(n + n_gen - 1, use_graph)
        torch.cuda.synchronize()
        return self.tokens[n:n + n_gen].tolist()
