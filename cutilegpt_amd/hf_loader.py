"""HuggingFace GPT-2 checkpoint I/O (local directories, no network).

The reference loads by model name through ``GPT2LMHeadModel.from_pretrained``
(``cutile_gpt/models/gpt.py:231-304``, ``cutile_gpt/utils/hf_loader.py:21-87``).
Here a local HF-format directory (``config.json`` + ``model.safetensors`` or
``pytorch_model.bin``) is read directly with safetensors / ``torch.load(...,
weights_only=True)``; a name that is not a directory goes to ``transformers``
(which needs its cache, since there is no network).

Key mapping (``cutile_gpt/models/gpt.py:255-299``): ``transformer.wte/wpe/h.i.*/
ln_f.*`` -> ``wte, wpe, h.i.*, ln_f.*``; HF Conv1D weights are (in, out) and are
transposed to the (out, in) layout the GEMM consumes; ``lm_head.weight`` is tied
to ``wte``.
"""

from __future__ import annotations

import json
import os
from typing import Any, Dict, Optional, Tuple

import torch

from .config import GPTConfig

_CONV1D = ("attn.c_attn.weight", "attn.c_proj.weight", "mlp.c_fc.weight", "mlp.c_proj.weight")
_PER_LAYER = ("ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias",
              "attn.c_proj.weight", "attn.c_proj.bias", "ln_2.weight", "ln_2.bias",
              "mlp.c_fc.weight", "mlp.c_fc.bias", "mlp.c_proj.weight", "mlp.c_proj.bias")


def config_from_hf(cfg: Dict[str, Any]) -> GPTConfig:
    """GPTConfig from an HF GPT-2 ``config.json`` dict."""
    return GPTConfig(vocab_size=cfg.get("vocab_size", 50257),
                     block_size=cfg.get("n_positions", cfg.get("n_ctx", 1024)),
                     n_layer=cfg["n_layer"], n_head=cfg["n_head"], n_embd=cfg["n_embd"])


def config_to_hf(config: GPTConfig) -> Dict[str, Any]:
    """HF GPT-2 ``config.json`` content for a GPTConfig (gelu_new, eps 1e-5, tied)."""
    return {
        "architectures": ["GPT2LMHeadModel"], "model_type": "gpt2",
        "vocab_size": config.vocab_size, "n_positions": config.block_size,
        "n_ctx": config.block_size, "n_embd": config.n_embd, "n_layer": config.n_layer,
        "n_head": config.n_head, "n_inner": None, "activation_function": "gelu_new",
        "layer_norm_epsilon": 1e-5, "resid_pdrop": 0.0, "embd_pdrop": 0.0, "attn_pdrop": 0.0,
        "tie_word_embeddings": True,
    }


def hf_to_internal(sd: Dict[str, torch.Tensor], n_layer: int) -> Dict[str, torch.Tensor]:
    """HF GPT-2 state_dict -> the reference's weight-dict layout (``gpt.py:255-299``)."""
    def get(key):
        for k in (key, key.replace("transformer.", "", 1)):
            if k in sd:
                return sd[k]
        raise KeyError(f"checkpoint has no {key}")

    w: Dict[str, torch.Tensor] = {"wte": get("transformer.wte.weight"),
                                  "wpe": get("transformer.wpe.weight")}
    for i in range(n_layer):
        for name in _PER_LAYER:
            t = get(f"transformer.h.{i}.{name}")
            w[f"h.{i}.{name}"] = t.t() if name in _CONV1D else t
    w["ln_f.weight"] = get("transformer.ln_f.weight")
    w["ln_f.bias"] = get("transformer.ln_f.bias")
    w["lm_head.weight"] = w["wte"]
    return w


def internal_to_hf(w: Dict[str, torch.Tensor], n_layer: int) -> Dict[str, torch.Tensor]:
    """Inverse of ``hf_to_internal`` (contiguous CPU tensors; lm_head tied)."""
    sd = {"transformer.wte.weight": w["wte"], "transformer.wpe.weight": w["wpe"]}
    for i in range(n_layer):
        for name in _PER_LAYER:
            t = w[f"h.{i}.{name}"]
            sd[f"transformer.h.{i}.{name}"] = t.t() if name in _CONV1D else t
    sd["transformer.ln_f.weight"] = w["ln_f.weight"]
    sd["transformer.ln_f.bias"] = w["ln_f.bias"]
    return {k: v.detach().cpu().contiguous() for k, v in sd.items()}


def save_hf_checkpoint(path: str, weights: Dict[str, torch.Tensor], config: GPTConfig) -> None:
    """Write ``config.json`` + ``model.safetensors`` in HF GPT-2 format."""
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(config_to_hf(config), f, indent=1)
    save_file(internal_to_hf(weights, config.n_layer), os.path.join(path, "model.safetensors"),
              metadata={"format": "pt"})


def load_hf_checkpoint(path: str, device: str = "cpu") -> Tuple[Dict[str, torch.Tensor], GPTConfig]:
    """Read an HF GPT-2 directory into (internal weight dict, GPTConfig).

    Tensors keep the checkpoint's dtype (a bf16 checkpoint is never widened on
    the host) and are read straight onto ``device``: safetensors files are
    loaded there by safetensors itself, ``pytorch_model.bin`` through
    ``torch.load(map_location=device, weights_only=True)``.  The Conv1D
    transposes are views; the model makes them contiguous on its device."""
    with open(os.path.join(path, "config.json")) as f:
        config = config_from_hf(json.load(f))
    st = os.path.join(path, "model.safetensors")
    if os.path.exists(st):
        from safetensors.torch import load_file
        sd = load_file(st, device=str(device))
    else:
        sd = torch.load(os.path.join(path, "pytorch_model.bin"), map_location=str(device),
                        weights_only=True)
    return hf_to_internal(sd, config.n_layer), config


class HFWeightLoader:
    """Load a GPT-2 checkpoint (mirrors ``cutile_gpt/utils/hf_loader.py:21-87``).

    ``load()`` returns ``(state_dict on the GPU, tokenizer or None)`` with the
    HF key names, like the reference.  ``model_name`` may be a local directory.
    """

    SUPPORTED_MODELS = {
        "gpt2": dict(n_layer=12, n_head=12, n_embd=768),
        "gpt2-medium": dict(n_layer=24, n_head=16, n_embd=1024),
        "gpt2-large": dict(n_layer=36, n_head=20, n_embd=1280),
        "gpt2-xl": dict(n_layer=48, n_head=25, n_embd=1600),
    }

    def __init__(self, model_name: str = "gpt2"):
        self.model_name = model_name
        self.config = self.SUPPORTED_MODELS.get(model_name, self.SUPPORTED_MODELS["gpt2"])
        self._tokenizer = None

    def load(self, device: str = "cuda") -> Tuple[Dict[str, torch.Tensor], Any]:
        if os.path.isdir(self.model_name):
            w, cfg = load_hf_checkpoint(self.model_name)
            self.config = dict(n_layer=cfg.n_layer, n_head=cfg.n_head, n_embd=cfg.n_embd)
            sd = internal_to_hf(w, cfg.n_layer)
            # GPT2LMHeadModel.state_dict() also lists the tied head.
            sd["lm_head.weight"] = sd["transformer.wte.weight"]
            # A tokenizer only when the directory holds its files (transformers
            # would otherwise build an empty one).
            self._tokenizer = None
            files = set(os.listdir(self.model_name))
            if "tokenizer.json" in files or {"vocab.json", "merges.txt"} <= files:
                from transformers import GPT2TokenizerFast
                self._tokenizer = GPT2TokenizerFast.from_pretrained(self.model_name)
        else:
            from transformers import GPT2LMHeadModel, GPT2Tokenizer
            model = GPT2LMHeadModel.from_pretrained(self.model_name)
            sd = model.state_dict()
            self._tokenizer = GPT2Tokenizer.from_pretrained(self.model_name)
        return {k: v.to(device) for k, v in sd.items()}, self._tokenizer

    @property
    def tokenizer(self):
        return self._tokenizer


def resolve_checkpoint(name_or_path: str, n_layer: Optional[int] = None, device: str = "cpu"):
    """Internal weight dict + GPTConfig for a local dir (read onto ``device``) or
    a cached HF name (CPU)."""
    if os.path.isdir(name_or_path):
        return load_hf_checkpoint(name_or_path, device)
    from transformers import GPT2LMHeadModel
    model = GPT2LMHeadModel.from_pretrained(name_or_path)
    c = model.config
    config = GPTConfig(vocab_size=c.vocab_size, block_size=c.n_positions, n_layer=c.n_layer,
                       n_head=c.n_head, n_embd=c.n_embd)
    return hf_to_internal(model.state_dict(), config.n_layer), config
