"""Qwen2 on the paged KV path (reference wrapper: python/llaisys/models/
qwen2.py:9-33, which is left unimplemented there).

The model runs in libllaisys (csrc/models/qwen2.cpp); this module loads
weights into the tensors the library hands out and marshals token arrays:

* `Qwen2(model_path)` reads `config.json` and `*.safetensors` from a local
  directory (HF Qwen2 names) and `generate()` decodes greedily, as the
  reference's `test/test_infer.py --test` compares (top_k=1);
* `Qwen2.random(meta, seed)` builds a random-init model of any Qwen2 shape on
  the GPU (bf16 weights ~ N(0, std), norm weights 1), for benchmarks and
  tests;
* `create_sequence / step / fork / free` drive the batched API: one step
  appends any number of tokens per sequence (prefill chunks and decodes
  mix) and returns each sequence's greedy next token; `decode` runs many
  greedy steps of a batch in one call.
"""
from __future__ import annotations

import json
from ctypes import POINTER, byref, c_int, c_int64, c_size_t
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import numpy as np

from ..libllaisys import LIB_LLAISYS, DataType, DeviceType, LlaisysQwen2Meta, check_last_error
from ..tensor import Tensor


@dataclass
class Qwen2Meta:
    nlayer: int
    hs: int
    nh: int
    nkvh: int
    di: int
    voc: int
    dh: int = 128
    maxseq: int = 4096
    epsilon: float = 1e-6
    theta: float = 10000.0
    end_token: int = -1
    dtype: DataType = DataType.BF16

    @classmethod
    def from_hf_config(cls, cfg: dict, maxseq: Optional[int] = None) -> "Qwen2Meta":
        nh = cfg["num_attention_heads"]
        eos = cfg.get("eos_token_id", -1)
        if isinstance(eos, list):
            eos = eos[0]
        return cls(
            nlayer=cfg["num_hidden_layers"],
            hs=cfg["hidden_size"],
            nh=nh,
            nkvh=cfg.get("num_key_value_heads", nh),
            di=cfg["intermediate_size"],
            voc=cfg["vocab_size"],
            dh=cfg.get("head_dim") or cfg["hidden_size"] // nh,
            maxseq=maxseq or min(cfg.get("max_position_embeddings", 4096), 32768),
            epsilon=cfg.get("rms_norm_eps", 1e-6),
            theta=cfg.get("rope_theta", 10000.0),
            end_token=-1 if eos is None else int(eos),
        )

    def c_struct(self) -> LlaisysQwen2Meta:
        return LlaisysQwen2Meta(int(self.dtype), self.nlayer, self.hs, self.nh, self.nkvh, self.dh, self.di,
                                self.maxseq, self.voc, self.epsilon, self.theta, self.end_token)


_LAYER_SLOTS = {  # HF name suffix -> LlaisysQwen2Weights field
    "input_layernorm.weight": "attn_norm_w",
    "self_attn.q_proj.weight": "attn_q_w",
    "self_attn.q_proj.bias": "attn_q_b",
    "self_attn.k_proj.weight": "attn_k_w",
    "self_attn.k_proj.bias": "attn_k_b",
    "self_attn.v_proj.weight": "attn_v_w",
    "self_attn.v_proj.bias": "attn_v_b",
    "self_attn.o_proj.weight": "attn_o_w",
    "post_attention_layernorm.weight": "mlp_norm_w",
    "mlp.gate_proj.weight": "mlp_gate_w",
    "mlp.up_proj.weight": "mlp_up_w",
    "mlp.down_proj.weight": "mlp_down_w",
}
_GLOBAL_SLOTS = {"model.embed_tokens.weight": "in_embed", "lm_head.weight": "out_embed", "model.norm.weight": "out_norm_w"}


class Qwen2:
    def __init__(self, model_path=None, device: DeviceType = DeviceType.AMD, *, meta: Qwen2Meta = None,
                 num_blocks: int = 0, device_id: int = 0):
        if model_path is not None:
            model_path = Path(model_path)
            cfg = json.loads((model_path / "config.json").read_text())
            meta = meta or Qwen2Meta.from_hf_config(cfg)
            tied = bool(cfg.get("tie_word_embeddings", False))
        if meta is None:
            raise ValueError("Qwen2 needs a model_path or a meta")
        self.meta = meta
        c_meta = meta.c_struct()
        ids = (c_int * 1)(device_id)
        if num_blocks:
            self._model = LIB_LLAISYS.llaisysQwen2ModelCreatePaged(byref(c_meta), int(device), ids, 1, num_blocks)
        else:
            self._model = LIB_LLAISYS.llaisysQwen2ModelCreate(byref(c_meta), int(device), ids, 1)
        check_last_error()
        self._weights = LIB_LLAISYS.llaisysQwen2ModelWeights(self._model).contents
        if model_path is not None:
            self._load_safetensors(model_path, tied)

    def __del__(self):
        if getattr(self, "_model", None):
            LIB_LLAISYS.llaisysQwen2ModelDestroy(self._model)
            self._model = None

    # ---- weights
    def weight_handle(self, name: str):
        """Library handle of an HF-named weight (owned by the model)."""
        if name in _GLOBAL_SLOTS:
            return getattr(self._weights, _GLOBAL_SLOTS[name])
        parts = name.split(".")
        if parts[:2] != ["model", "layers"]:
            raise KeyError(name)
        layer, suffix = int(parts[2]), ".".join(parts[3:])
        return getattr(self._weights, _LAYER_SLOTS[suffix])[layer]

    def weight_names(self) -> List[str]:
        names = list(_GLOBAL_SLOTS)
        for i in range(self.meta.nlayer):
            names += [f"model.layers.{i}.{s}" for s in _LAYER_SLOTS]
        return names

    def weight_shape(self, name: str) -> tuple:
        """Shape of an HF-named weight as the model holds it."""
        h = self.weight_handle(name)
        n = int(LIB_LLAISYS.tensorGetNdim(h))
        buf = (c_size_t * max(n, 1))()
        LIB_LLAISYS.tensorGetShape(h, buf)
        return tuple(int(buf[i]) for i in range(n))

    def load_weight(self, name: str, host_ptr: int, shape=None):
        """tensorLoad of contiguous host data (the weight's own dtype and shape).
        tensorLoad copies as many bytes as the weight holds; pass the source's
        `shape` to have a mismatch refused before anything is read."""
        if shape is not None and tuple(shape) != self.weight_shape(name):
            raise ValueError(f"{name}: source shape {tuple(shape)} does not match the model's "
                             f"{self.weight_shape(name)}")
        LIB_LLAISYS.tensorLoad(self.weight_handle(name), host_ptr)
        check_last_error()

    def _load_safetensors(self, model_path: Path, tied: bool):
        import safetensors
        import torch

        seen = set()
        for file in sorted(model_path.glob("*.safetensors")):
            with safetensors.safe_open(file, framework="pt", device="cpu") as f:
                for name in f.keys():
                    if name not in _GLOBAL_SLOTS and ".".join(name.split(".")[3:]) not in _LAYER_SLOTS:
                        continue
                    t = f.get_tensor(name).to(torch.bfloat16).contiguous()
                    self.load_weight(name, t.data_ptr(), t.shape)
                    seen.add(name)
                    if tied and name == "model.embed_tokens.weight":
                        self.load_weight("lm_head.weight", t.data_ptr(), t.shape)
                        seen.add("lm_head.weight")
        missing = [n for n in self.weight_names() if n not in seen]
        if missing:
            raise ValueError(f"{len(missing)} weights missing from {model_path}, e.g. {missing[:3]}")

    @classmethod
    def random(cls, meta: Qwen2Meta, seed: int = 0, std: float = 0.02, num_blocks: int = 0, device_id: int = 0):
        """Random-init weights ~ N(0, std) in bf16 (norm weights 1), made on the GPU."""
        import torch

        from ..libllaisys import MemcpyKind
        from ..runtime import RuntimeAPI

        model = cls(meta=meta, num_blocks=num_blocks, device_id=device_id)
        api = RuntimeAPI(DeviceType.AMD)
        g = torch.Generator(device=f"cuda:{device_id}").manual_seed(seed)
        for name in model.weight_names():
            h = model.weight_handle(name)
            t = Tensor(tensor=h)
            try:
                shape = t.shape()
                if name.endswith("norm.weight"):
                    src = torch.ones(shape, dtype=torch.bfloat16, device=f"cuda:{device_id}")
                else:
                    src = torch.empty(shape, dtype=torch.bfloat16, device=f"cuda:{device_id}").normal_(0.0, std, generator=g)
                api.memcpy_sync(t.data_ptr(), src.data_ptr(), src.numel() * 2, MemcpyKind.D2D)
            finally:
                t._tensor = None  # borrowed handle: the model owns it
        return model

    # ---- single sequence (reference API)
    def infer(self, tokens: Sequence[int]) -> int:
        arr = (c_int64 * len(tokens))(*tokens)
        nxt = LIB_LLAISYS.llaisysQwen2ModelInfer(self._model, arr, len(tokens))
        check_last_error()
        return int(nxt)

    def generate(self, inputs: Sequence[int], max_new_tokens: int = None, top_k: int = 1, top_p: float = 0.8,
                 temperature: float = 0.8) -> List[int]:
        """Greedy decoding (the sampling arguments of the reference signature
        are accepted; tokens are argmax, as test_infer.py --test compares).
        Returns inputs + generated tokens, like HF generate."""
        out = list(inputs)
        max_new_tokens = 128 if max_new_tokens is None else max_new_tokens
        for _ in range(max_new_tokens):
            nxt = self.infer(out)
            out.append(nxt)
            if nxt == self.meta.end_token:
                break
        return out

    # ---- batched sequences
    def create_sequence(self, tokens: Sequence[int] = None):
        """Returns (seq_id, reused): reused leading tokens are already cached."""
        reused = c_size_t(0)
        if tokens:
            arr = (c_int64 * len(tokens))(*tokens)
            sid = LIB_LLAISYS.llaisysQwen2SeqCreate(self._model, arr, len(tokens), byref(reused))
        else:
            sid = LIB_LLAISYS.llaisysQwen2SeqCreate(self._model, None, 0, byref(reused))
        check_last_error()
        return int(sid), int(reused.value)

    def fork(self, seq_id: int) -> int:
        sid = LIB_LLAISYS.llaisysQwen2SeqFork(self._model, seq_id)
        check_last_error()
        return int(sid)

    def free(self, seq_id: int):
        LIB_LLAISYS.llaisysQwen2SeqFree(self._model, seq_id)
        check_last_error()

    def length(self, seq_id: int) -> int:
        n = LIB_LLAISYS.llaisysQwen2SeqLength(self._model, seq_id)
        check_last_error()
        return int(n)

    def num_free_blocks(self) -> int:
        return int(LIB_LLAISYS.llaisysQwen2NumFreeBlocks(self._model))

    def warm_up(self, max_tokens: int = 256):
        """Run one throwaway step of b single-token sequences for b = 1, 2, 4,
        ... up to max_tokens (and the free blocks), so the step workspaces
        reach their serving sizes before serving, instead of growing inside
        the first step that meets each size."""
        b = 1
        while b <= min(max_tokens, self.num_free_blocks()):
            ids = [self.create_sequence()[0] for _ in range(b)]
            try:
                self.step(ids, [[0]] * b)
            finally:
                for i in ids:
                    self.free(i)
            b *= 2

    def step(self, seq_ids: Sequence[int], tokens: Sequence[Sequence[int]]) -> List[int]:
        """Append tokens[i] to sequence seq_ids[i]; returns each greedy next token."""
        B = len(seq_ids)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(t, dtype=np.int64) for t in tokens]))
        counts = (c_size_t * B)(*[len(t) for t in tokens])
        ids = (c_int64 * B)(*seq_ids)
        nxt = (c_int64 * B)()
        LIB_LLAISYS.llaisysQwen2ModelStep(self._model, ids, B, flat.ctypes.data_as(POINTER(c_int64)), counts, nxt)
        check_last_error()
        return list(nxt)

    def step_arrays(self, seq_ids: np.ndarray, flat_tokens: np.ndarray, counts: np.ndarray, out: np.ndarray):
        """step() over prepared int64 / size_t numpy arrays (no Python lists)."""
        LIB_LLAISYS.llaisysQwen2ModelStep(
            self._model, seq_ids.ctypes.data_as(POINTER(c_int64)), seq_ids.size,
            flat_tokens.ctypes.data_as(POINTER(c_int64)), counts.ctypes.data_as(POINTER(c_size_t)),
            out.ctypes.data_as(POINTER(c_int64)))
        check_last_error()

    def decode(self, seq_ids: Sequence[int], first_tokens: Sequence[int], nsteps: int) -> np.ndarray:
        """nsteps greedy steps in one call (tokens fed back on the device).
        Returns int64 [nsteps, nseq]: row s = each sequence's token after step s."""
        ids = np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int64))
        first = np.ascontiguousarray(np.asarray(first_tokens, dtype=np.int64))
        out = np.zeros((nsteps, ids.size), np.int64)
        LIB_LLAISYS.llaisysQwen2ModelDecode(self._model, ids.ctypes.data_as(POINTER(c_int64)), ids.size,
                                            first.ctypes.data_as(POINTER(c_int64)), nsteps,
                                            out.ctypes.data_as(POINTER(c_int64)))
        check_last_error()
        return out

    def logits(self) -> Tensor:
        """[nseq, voc] logits of the last infer/step (a view; copy before the next call)."""
        h = LIB_LLAISYS.llaisysQwen2ModelLogits(self._model)
        check_last_error()
        return Tensor(tensor=h)
