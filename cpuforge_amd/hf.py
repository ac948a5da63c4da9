"""LoRA adapter files (crates/io/src/hf.rs:60-179), read into and written from
device-resident adapters:

    save_adapter(path, model)                    hf.rs:60-75   one safetensors file
    load_adapter(model, path)                    hf.rs:146-179
    save_peft_adapter(dir, model, base_model)    hf.rs:82-106  adapter_config.json +
                                                               adapter_model.safetensors
    load_peft_adapter(model, dir)                hf.rs:109-143

The model protocol is that of `cpuforge_amd.state` (`named_params`,
`lora_cfg`, `add_lora`); LoRA tensors are the parameters whose name holds
".lora_".  Errors raise `FormatError` with the reference's message.
"""
from __future__ import annotations

import json
import os

import torch

from .st import FormatError, read_safetensors, write_safetensors
from .state import json_f64, lora_meta, parse_f32, parse_u64


def _lora_params(model):
    return [(n, p) for n, p in model.named_params() if ".lora_" in n]


def _os_error(e: OSError) -> str:
    return f"{e.strerror} (os error {e.errno})" if e.errno else str(e)


def save_adapter(path, model) -> None:
    """hf.rs:60-75: the LoRA tensors under their own names, with the
    rank / alpha / targets metadata that rebuilds the adapter structure."""
    lc = model.lora_cfg
    if lc is None:
        raise FormatError("model has no LoRA adapters")
    owned = [(n, list(p.shape), p.detach()) for n, p in _lora_params(model)]
    write_safetensors(path, owned, lora_meta(lc))


def _fill(model, loaded, key_of) -> None:
    seen = 0
    with torch.no_grad():
        for name, p in _lora_params(model):
            key = key_of(name)
            t = loaded.tensors.get(key)
            if t is None:
                raise FormatError(f"adapter file is missing '{key}'")
            if list(t.shape) != list(p.shape):
                raise FormatError(f"adapter tensor '{key}' has shape {list(t.shape)}, expected {list(p.shape)}")
            p.copy_(t)
            seen += 1
    if seen != len(loaded.tensors):
        raise FormatError(f"adapter file has {len(loaded.tensors)} tensors but the model uses {seen}")


def load_adapter(model, path) -> None:
    """hf.rs:146-179: attaches adapters from the file's metadata and fills
    them from its tensors."""
    loaded = read_safetensors(path)

    def get(k):
        if k not in loaded.metadata:
            raise FormatError(f"adapter file lacks metadata '{k}'")
        return loaded.metadata[k]

    rank = parse_u64(get("lora_rank"))
    if rank is None:
        raise FormatError("bad lora_rank")
    alpha = parse_f32(get("lora_alpha"))
    if alpha is None:
        raise FormatError("bad lora_alpha")
    targets = [s for s in get("lora_targets").split(",") if s]
    model.add_lora(rank, float(alpha), targets, 0)
    _fill(model, loaded, lambda n: n)


def _pretty(obj: dict) -> str:
    """serde_json::to_string_pretty of a json! object: keys in byte order
    (serde_json's Map is a BTreeMap), two-space indent, no final newline."""
    lines = []
    for k in sorted(obj, key=lambda s: s.encode()):
        v = obj[k]
        if isinstance(v, bool):
            s = "true" if v else "false"
        elif isinstance(v, int):
            s = str(v)
        elif isinstance(v, float):
            s = json_f64(v)
        elif isinstance(v, str):
            s = json.dumps(v, ensure_ascii=False)
        elif isinstance(v, list):
            s = "[]" if not v else "[\n" + ",\n".join("    " + json.dumps(x, ensure_ascii=False) for x in v) + "\n  ]"
        else:
            raise TypeError(k)
        lines.append(f"  {json.dumps(k, ensure_ascii=False)}: {s}")
    return "{\n" + ",\n".join(lines) + "\n}"


def save_peft_adapter(dir_, model, base_model: str) -> None:
    """hf.rs:82-106: `adapter_model.safetensors` with PEFT's tensor names
    (base_model.model.<name>.weight, metadata format=pt) and
    `adapter_config.json` with PEFT's LoRA fields."""
    lc = model.lora_cfg
    if lc is None:
        raise FormatError("model has no LoRA adapters")
    try:
        os.makedirs(dir_, exist_ok=True)
    except OSError as e:
        raise FormatError(f"cannot create {dir_}: {_os_error(e)}") from None
    owned = [(f"base_model.model.{n}.weight", list(p.shape), p.detach()) for n, p in _lora_params(model)]
    write_safetensors(os.path.join(dir_, "adapter_model.safetensors"), owned, {"format": "pt"})
    cfg = {"peft_type": "LORA", "task_type": "CAUSAL_LM", "base_model_name_or_path": base_model, "r": int(lc.rank),
           "lora_alpha": float(torch.tensor(lc.alpha, dtype=torch.float32).item()), "lora_dropout": 0.0,
           "bias": "none", "target_modules": [f"{t}_proj" for t in lc.targets], "fan_in_fan_out": False,
           "inference_mode": True, "use_rslora": False, "use_dora": False}
    try:
        with open(os.path.join(dir_, "adapter_config.json"), "w", encoding="utf-8") as fh:
            fh.write(_pretty(cfg))
    except OSError as e:
        raise FormatError(_os_error(e)) from None


def load_peft_adapter(model, dir_) -> None:
    """hf.rs:109-143: attaches LoRA adapters described by a PEFT directory
    (LoRA only; DoRA and rsLoRA refused) and fills them."""
    try:
        with open(os.path.join(dir_, "adapter_config.json"), encoding="utf-8") as fh:
            text = fh.read()
    except OSError as e:
        raise FormatError(f"cannot read adapter_config.json in {dir_}: {_os_error(e)}") from None
    try:
        cfg = json.loads(text)
    except ValueError as e:
        raise FormatError(f"bad adapter_config.json: {e}") from None
    if not isinstance(cfg, dict):
        cfg = {}
    if cfg.get("peft_type") != "LORA":
        raise FormatError("only LoRA adapters are supported")
    if cfg.get("use_dora") is True or cfg.get("use_rslora") is True:
        raise FormatError("DoRA / rsLoRA adapters are not supported")
    r = cfg.get("r")
    if not (isinstance(r, int) and not isinstance(r, bool) and 0 <= r < 2 ** 64):
        raise FormatError("adapter_config.json lacks r")
    alpha = cfg.get("lora_alpha")
    if not (isinstance(alpha, (int, float)) and not isinstance(alpha, bool)):
        raise FormatError("adapter_config.json lacks lora_alpha")
    mods = cfg.get("target_modules")
    if not isinstance(mods, list):
        raise FormatError("adapter_config.json lacks target_modules")
    targets = [m[:-5] if m.endswith("_proj") else m for m in mods if isinstance(m, str)]
    model.add_lora(r, float(torch.tensor(float(alpha), dtype=torch.float32).item()), targets, 0)
    loaded = read_safetensors(os.path.join(dir_, "adapter_model.safetensors"))
    _fill(model, loaded, lambda n: f"base_model.model.{n}.weight")
