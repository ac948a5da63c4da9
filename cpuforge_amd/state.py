"""Resumable training state in one safetensors file (crates/train/src/state.rs),
written from and restored into device-resident parameters and AdamW moments.

    save_state(path, model, opt, step, consumed)   state.rs:14-52
    load_state(path, model, opt) -> (step, consumed)  state.rs:56-102

Tensors are stored as `p.<name>`, `m.<name>`, `v.<name>` for every parameter
that trains, with the metadata "step", "consumed", "opt_step" and, when the
model has LoRA adapters, "lora_rank", "lora_alpha", "lora_targets".  A model
is any object with `named_params()` (visit_params order,
crates/model/src/model.rs:179-208), `lora_cfg` (None or rank / alpha /
targets) and `add_lora(rank, alpha, targets, seed)`; the optimizer is
`cpuforge_amd.optim.AdamW`.  Errors raise `FormatError` with the reference's
message.
"""
from __future__ import annotations

import math
import re

import numpy as np
import torch

from .st import FormatError, read_safetensors, write_safetensors


def rust_f32_str(x: float) -> str:
    """`f32`'s Display in Rust (what `alpha.to_string()` writes): the shortest
    decimal that reads back as the same f32, positional, no trailing ".0"."""
    x = np.float32(x)
    if np.isnan(x):
        return "NaN"
    if np.isinf(x):
        return "inf" if x > 0 else "-inf"
    return np.format_float_positional(x, unique=True, trim="-")


def parse_u64(s: str):
    """Rust's `str::parse::<u64>()`: an optional '+' and decimal digits only;
    None where Rust returns Err."""
    if not re.fullmatch(r"\+?[0-9]+", s):
        return None
    v = int(s)
    return v if v < 2 ** 64 else None


def parse_f32(s: str):
    """Rust's `str::parse::<f32>()` for the decimal forms it accepts; None
    where it returns Err."""
    if re.fullmatch(r"[+-]?(inf|infinity|nan)", s, flags=re.I):
        return np.float32(float(s))
    if not re.fullmatch(r"[+-]?([0-9]+\.?[0-9]*|\.[0-9]+)([eE][+-]?[0-9]+)?", s):
        return None
    return np.float32(float(s))


def lora_meta(lc) -> dict:
    return {"lora_rank": str(lc.rank), "lora_alpha": rust_f32_str(lc.alpha), "lora_targets": ",".join(lc.targets)}


def save_state(path, model, opt, step: int, consumed: int) -> None:
    """state.rs:14-52.  Parameters without a gradient are not stored; a
    parameter the optimizer has not touched yet gets zero moments."""
    owned = []
    for name, p in model.named_params():
        if not p.requires_grad:
            continue
        shape = list(p.shape)
        owned.append((f"p.{name}", shape, p.detach()))
        if name in opt.state:
            m, v = opt.state[name]
        else:
            m = v = torch.zeros_like(p)
        owned.append((f"m.{name}", shape, m))
        owned.append((f"v.{name}", shape, v))
    meta = {"step": str(step), "consumed": str(consumed), "opt_step": str(opt.step)}
    if model.lora_cfg is not None:
        meta.update(lora_meta(model.lora_cfg))
    write_safetensors(path, owned, meta)


def load_state(path, model, opt):
    """state.rs:56-102: restores the saved parameters into `model` (attaching
    the file's LoRA adapters first when the model has none), replaces the
    optimizer's moments and step count, and returns (step, consumed)."""
    loaded = read_safetensors(path)
    meta = loaded.metadata

    def num(k):
        if k not in meta:
            raise FormatError(f"state file lacks '{k}'")
        v = parse_u64(meta[k])
        if v is None:
            raise FormatError(f"bad '{k}' in state file")
        return v

    if "lora_rank" in meta:
        rank = parse_u64(meta["lora_rank"])
        if rank is None:
            raise FormatError("bad lora_rank")
        if "lora_alpha" not in meta:
            raise FormatError("state file lacks lora_alpha")
        alpha = parse_f32(meta["lora_alpha"])
        if alpha is None:
            raise FormatError("bad lora_alpha")
        targets = [s for s in meta.get("lora_targets", "").split(",") if s]
        lc = model.lora_cfg
        if lc is None:
            model.add_lora(rank, float(alpha), targets, 0)
        elif not (lc.rank == rank and np.float32(lc.alpha) == alpha and list(lc.targets) == targets):
            raise FormatError("model's LoRA setup differs from the one in the state file")

    restored, new_state = 0, {}
    with torch.no_grad():
        for name, p in model.named_params():
            t = loaded.tensors.get(f"p.{name}")
            if t is None:
                continue
            if list(t.shape) != list(p.shape):
                raise FormatError(f"'{name}' has shape {list(t.shape)} in the state file, expected {list(p.shape)}")
            p.copy_(t)
            restored += 1
            m, v = loaded.tensors.get(f"m.{name}"), loaded.tensors.get(f"v.{name}")
            if m is not None and v is not None:
                new_state[name] = (m, v)
    in_file = sum(1 for k in loaded.tensors if k.startswith("p."))
    if restored != in_file:
        raise FormatError(f"state file has {in_file} parameter tensors but only {restored} matched this model")
    opt.state = new_state
    opt.step = num("opt_step")
    return num("step"), num("consumed")


def json_f64(x: float) -> str:
    """serde_json's text of an f64 (its ryu formatter): the shortest
    round-trip digits d_1..d_n with the decimal point after kk digits, then
      integral with kk <= 16       -> digits, zeros, ".0"   (1e15 -> "1000000000000000.0")
      0 < kk <= 16                 -> "123.456"
      -5 < kk <= 0                 -> "0.00005"
      otherwise                    -> "1e-7", "1.5e16";
    non-finite values are null."""
    if not math.isfinite(x):
        return "null"
    r = repr(float(x))
    sign = "-" if r.startswith("-") else ""
    r = r.lstrip("-")
    mant, exp = (r.split("e") + ["0"])[:2]
    ip, fp = (mant.split(".") + [""])[:2]
    full = ip + fp
    z = len(full) - len(full.lstrip("0"))
    digits = full[z:].rstrip("0")
    if not digits:
        return sign + "0.0"
    kk = len(ip) - z + int(exp)  # value = 0.digits * 10**kk
    n = len(digits)
    if kk - n >= 0 and kk <= 16:
        return sign + digits + "0" * (kk - n) + ".0"
    if 0 < kk <= 16:
        return sign + digits[:kk] + "." + digits[kk:]
    if -5 < kk <= 0:
        return sign + "0." + "0" * (-kk) + digits
    if n == 1:
        return f"{sign}{digits}e{kk - 1}"
    return f"{sign}{digits[0]}.{digits[1:]}e{kk - 1}"
