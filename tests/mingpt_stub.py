"""A stand-in for a minGPT module (test helper): carries a minGPT state_dict,
nn.Linear (out, in) weights under ``transformer.*`` and a separate
``lm_head.weight`` (minGPT does not tie it), for ``CutileGPT.load_from_mingpt``
(reference: cutile_gpt/models/gpt.py:306-343)."""

import torch


class MinGPTStub(torch.nn.Module):
    def __init__(self, w, n_layer):
        super().__init__()
        self._sd = {"transformer.wte.weight": w["wte"], "transformer.wpe.weight": w["wpe"],
                    "transformer.ln_f.weight": w["ln_f.weight"],
                    "transformer.ln_f.bias": w["ln_f.bias"], "lm_head.weight": w["lm_head.weight"]}
        for i in range(n_layer):
            for k, v in w.items():
                if k.startswith(f"h.{i}."):
                    self._sd["transformer." + k] = v

    def state_dict(self, *args, **kwargs):
        return dict(self._sd)
