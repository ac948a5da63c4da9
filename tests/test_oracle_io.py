"""CPU tests of the on-disk formats (no GPU needed).

- The oracle's bf16 / f16 conversions against the reference's known-answer
  tests (crates/io/src/dtype.rs:36-57) and, over all 65536 patterns, against
  numpy's half-precision conversion (an independent implementation).
- The library's safetensors header reader (cfio_st_open, host code) against
  files written by the `safetensors` Python package 0.8.0, which wraps the
  same Rust crate version as the reference's Cargo.lock:1177-1178: names,
  dtypes, shapes and metadata, and, for malformed files, the crate's own
  verdict and message (the reference reports "PATH: <crate message>",
  crates/io/src/st.rs:26-32).
- The Rust formatting helpers of the state and adapter files.
"""
import json
import struct

import numpy as np
import pytest

from cpuforge_amd import hf, state
from cpuforge_amd.st import FormatError, StFile
from oracle import oracle as O

safetensors = pytest.importorskip("safetensors")
from safetensors.numpy import save as st_save  # noqa: E402


# ---------------------------------------------------------------- dtype.rs
def test_f16_known_values():
    """dtype.rs:40-50."""
    got = O.f16_to_f32(np.array([0x3C00, 0xC000, 0x0000, 0x7BFF, 0x0400, 0x0001, 0x03FF], np.uint16))
    want = [1.0, -2.0, 0.0, 65504.0, 2.0 ** -14, 2.0 ** -24, 1023.0 * 2.0 ** -24]
    assert got.tolist() == want
    inf_nan = O.f16_to_f32(np.array([0x7C00, 0x7E00], np.uint16))
    assert np.isinf(inf_nan[0]) and np.isnan(inf_nan[1])
    assert O.f16_to_f32(np.array([0x3555], np.uint16))[0] == np.float32(0.33325195)


def test_bf16_known_values():
    """dtype.rs:53-57."""
    got = O.bf16_to_f32(np.array([0x3F80, 0xC000, 0x0000, 0x4049], np.uint16))
    assert got.tolist() == [1.0, -2.0, 0.0, 3.140625]


def test_f16_all_patterns_match_numpy_bitwise():
    bits = np.arange(65536, dtype=np.uint16)
    got = O.f16_to_f32(bits).view(np.uint32)
    want = bits.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got, want)


def test_bf16_all_patterns_are_the_high_half():
    bits = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(O.bf16_to_f32(bits).view(np.uint32), bits.astype(np.uint32) << 16)


def test_a_planted_f16_mistake_is_caught():
    """The exhaustive comparison fails for a conversion that drops the
    subnormal renormalisation (a plausible restatement slip)."""
    bits = np.arange(65536, dtype=np.uint16)
    sign, exp, man = (bits >> 15).astype(np.uint32), ((bits >> 10) & 0x1F).astype(np.uint32), (bits & 0x3FF).astype(np.uint32)
    wrong = np.where(exp == 0, sign << 31, (sign << 31) | ((exp + 112) << 23) | (man << 13)).astype(np.uint32)
    wrong = np.where(exp == 0x1F, (sign << 31) | (0xFF << 23) | (man << 13), wrong).astype(np.uint32)
    want = bits.view(np.float16).astype(np.float32).view(np.uint32)
    assert not np.array_equal(wrong, want)


# ---------------------------------------------------------------- header reader
def _write(tmp_path, name, data: bytes):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_reader_agrees_with_the_crate_on_every_dtype(tmp_path):
    import torch
    from safetensors.torch import save as tsave
    dts = {"bool": torch.bool, "u8": torch.uint8, "i8": torch.int8, "e5m2": torch.float8_e5m2,
           "e4m3": torch.float8_e4m3fn, "i16": torch.int16, "u16": torch.uint16, "f16": torch.float16,
           "bf16": torch.bfloat16, "i32": torch.int32, "u32": torch.uint32, "f32": torch.float32,
           "f64": torch.float64, "i64": torch.int64, "u64": torch.uint64, "c64": torch.complex64}
    for extra in ("float8_e8m0fnu",):
        if hasattr(torch, extra):
            dts[extra] = getattr(torch, extra)
    ts = {k: torch.zeros(3, 2, dtype=d) for k, d in dts.items()}
    ts["scalar"] = torch.tensor(3.0)
    ts["empty"] = torch.zeros(0, 5)
    data = tsave(ts, metadata={"step": "42", "k": "v"})
    path = _write(tmp_path, "all.safetensors", data)
    n = int.from_bytes(data[:8], "little")
    hdr = json.loads(data[8:8 + n])
    with StFile(path) as f:
        got = {name: (dt, shape) for name, dt, shape, _ in f.tensors()}
        offsets = [hdr[name]["data_offsets"] for name, _, _, _ in f.tensors()]
        assert f.metadata() == {"step": "42", "k": "v"}
    want = {k: (v["dtype"], v["shape"]) for k, v in hdr.items() if k != "__metadata__"}
    assert got == want
    assert offsets == sorted(offsets)  # file order


def test_reader_decodes_escaped_and_unicode_names(tmp_path):
    names = ['a"\\\n\x01\x7fé/', "☃ snow", "tab\there", "emoji \U0001F600"]
    data = st_save({n: np.zeros(2, np.float32) for n in names})
    path = _write(tmp_path, "names.safetensors", data)
    with StFile(path) as f:
        assert sorted(n for n, _, _, _ in f.tensors()) == sorted(names)
    # \u escapes with a surrogate pair, written by hand
    h = '{"\\ud83d\\ude00x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}'
    path = _write(tmp_path, "esc.safetensors", struct.pack("<Q", len(h)) + h.encode() + b"\0" * 4)
    with StFile(path) as f:
        assert f.tensors()[0][0] == "\U0001F600x"


def _crate_verdict(path):
    from safetensors import safe_open
    try:
        with safe_open(path, "np"):
            return None
    except Exception as e:  # the binding's SafetensorError
        msg = str(e)
        prefix = "Error while deserializing header: "
        return msg[len(prefix):] if msg.startswith(prefix) else msg


def _mk(h, data=b"", n=None):
    hb = h.encode() if isinstance(h, str) else h
    return struct.pack("<Q", len(hb) if n is None else n) + hb + data


MALFORMED = {
    "small": b"\x01\x02",
    "toolarge": struct.pack("<Q", 100_000_001) + b"{}",
    "badlen": _mk("{}", n=50),
    "badstart": _mk("[1]"),
    "badjson": _mk('{"a":'),
    "badutf8": _mk(b'{"\xff":1}'),
    "badutf8_3": _mk(b'{"\xe2\x82":1}'),
    "gap": _mk(json.dumps({"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}), b"\0" * 8),
    "info": _mk(json.dumps({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}), b"\0" * 4),
    "incomplete": _mk(json.dumps({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}), b"\0" * 8),
    "unkdtype": _mk(json.dumps({"a": {"dtype": "F17", "shape": [1], "data_offsets": [0, 4]}}), b"\0" * 4),
    "overflow": _mk(json.dumps({"a": {"dtype": "F32", "shape": [2 ** 40, 2 ** 40], "data_offsets": [0, 4]}}),
                    b"\0" * 4),
    "f4odd": _mk(json.dumps({"a": {"dtype": "F4", "shape": [3], "data_offsets": [0, 2]}}), b"\0" * 2),
    "metanum": _mk(json.dumps({"__metadata__": {"a": 1}})),
    "negshape": _mk(json.dumps({"a": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}), b"\0" * 4),
    "missing": _mk(json.dumps({"a": {"dtype": "F32", "shape": [1]}}), b"\0" * 4),
    "trail": _mk("{} x"),
    "dup": _mk('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},'
               '"a":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}', b"\0" * 8),
    "three": _mk(json.dumps({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4, 8]}}), b"\0" * 8),
    "float": _mk(json.dumps({"a": {"dtype": "F32", "shape": [1.0], "data_offsets": [0, 4]}}), b"\0" * 4),
    "overlap": _mk(json.dumps({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
                               "b": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}), b"\0" * 8),
    "backwards": _mk(json.dumps({"a": {"dtype": "F32", "shape": [0], "data_offsets": [4, 0]}}), b"\0" * 4),
    "empty": b"",
}
ACCEPTED = {
    "metanull": _mk(json.dumps({"__metadata__": None})),
    "extra": _mk(json.dumps({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4], "zz": [1, {"q": None}]}}),
                 b"\0" * 4),
    "spaces": _mk('  { "a" : { "shape" : [ 1 ] , "data_offsets" : [ 0 , 4 ] , "dtype" : "F32" } }   ', b"\0" * 4),
    "zero_sized": _mk(json.dumps({"z": {"dtype": "F32", "shape": [0, 3], "data_offsets": [0, 0]},
                                  "a": {"dtype": "BF16", "shape": [1], "data_offsets": [0, 2]}}), b"\0" * 2),
}


@pytest.mark.parametrize("case", sorted(MALFORMED))
def test_malformed_files_fail_as_the_crate_fails(tmp_path, case):
    path = _write(tmp_path, case, MALFORMED[case])
    crate = _crate_verdict(path)
    assert crate is not None
    with pytest.raises(FormatError) as e:
        StFile(path)
    ours = str(e.value)
    assert ours.startswith(path + ": ")
    ours = ours[len(path) + 2:]
    if crate.startswith("invalid JSON in header"):
        # serde_json's wording of the parse error (with its line / column) is
        # not restated; the crate's category is.
        assert ours.startswith("invalid JSON in header: "), ours
    else:
        assert ours == crate


@pytest.mark.parametrize("case", sorted(ACCEPTED))
def test_files_the_crate_accepts_are_accepted(tmp_path, case):
    path = _write(tmp_path, case, ACCEPTED[case])
    assert _crate_verdict(path) is None
    with StFile(path) as f:
        f.tensors()


def test_duplicate_names_keep_the_last_record(tmp_path):
    h = ('{"a":{"dtype":"F32","shape":[9],"data_offsets":[0,36]},'
         '"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}')
    path = _write(tmp_path, "dup_ok", _mk(h, b"\0" * 4))
    assert _crate_verdict(path) is None
    with StFile(path) as f:
        assert f.tensors() == [("a", "F32", [1], 1)]


def test_missing_file_and_directory(tmp_path):
    missing = str(tmp_path / "nope")
    with pytest.raises(FormatError) as e:
        StFile(missing)
    assert str(e.value) == f"cannot open {missing}: No such file or directory (os error 2)"
    with pytest.raises(FormatError):
        StFile(str(tmp_path))


# ---------------------------------------------------------------- Rust text formats
def test_rust_f32_display():
    """`f32::to_string`: shortest round-trip digits, no exponent, no ".0"."""
    cases = {32.0: "32", 8.0: "8", 6.0: "6", 0.5: "0.5", 0.1: "0.1", 1e-8: "0.00000001", 16.5: "16.5",
             1e10: "10000000000", -0.0: "-0", 3.4028234663852886e38: "340282350000000000000000000000000000000",
             float("inf"): "inf", float("nan"): "NaN"}
    for x, s in cases.items():
        assert state.rust_f32_str(x) == s, x
    for s in ("32", "0.1", "1e-8", "+2.5", ".5", "5.", "inf", "NaN"):
        assert state.parse_f32(s) is not None
    for s in ("", "x", "1_0", " 1", "0x10", "1e"):
        assert state.parse_f32(s) is None
    assert state.parse_f32("0.1") == np.float32(0.1)


def test_rust_u64_parse():
    assert state.parse_u64("42") == 42 and state.parse_u64("+7") == 7
    for s in ("", "-1", " 1", "1_0", "1.0", str(2 ** 64)):
        assert state.parse_u64(s) is None
    assert state.parse_u64(str(2 ** 64 - 1)) == 2 ** 64 - 1


def test_json_f64_matches_serde_json_text():
    assert state.json_f64(6.0) == "6.0"
    assert state.json_f64(0.0) == "0.0"
    assert state.json_f64(float(np.float32(0.1))) == "0.10000000149011612"
    assert state.json_f64(1e-7) == "1e-7"
    assert state.json_f64(float("nan")) == "null"
    # ryu keeps the decimal form down to 1e-5 (Python's repr leaves it at 1e-4)
    assert state.json_f64(5e-5) == "0.00005"
    assert state.json_f64(1.5e-5) == "0.000015"
    assert state.json_f64(1e-5) == "0.00001"
    assert state.json_f64(1e-6) == "1e-6"
    assert state.json_f64(1.5e-6) == "1.5e-6"
    assert state.json_f64(0.0001) == "0.0001"
    assert state.json_f64(1e15) == "1000000000000000.0"
    assert state.json_f64(1e16) == "1e16"
    assert state.json_f64(1.5e16) == "1.5e16"
    assert state.json_f64(123456.789) == "123456.789"
    assert state.json_f64(-2.5) == "-2.5"
    assert state.json_f64(-0.0) == "-0.0"
    assert state.json_f64(1.7976931348623157e308) == "1.7976931348623157e308"
    assert state.json_f64(5e-324) == "5e-324"


def test_peft_config_text_is_serde_pretty_with_sorted_keys():
    """hf.rs:95-103 through serde_json::to_string_pretty: BTreeMap key
    order, two-space indent, one array element per line."""
    cfg = {"peft_type": "LORA", "task_type": "CAUSAL_LM", "base_model_name_or_path": "org/base", "r": 3,
           "lora_alpha": 6.0, "lora_dropout": 0.0, "bias": "none", "target_modules": ["q_proj", "v_proj"],
           "fan_in_fan_out": False, "inference_mode": True, "use_rslora": False, "use_dora": False}
    text = hf._pretty(cfg)
    assert text == (
        '{\n  "base_model_name_or_path": "org/base",\n  "bias": "none",\n  "fan_in_fan_out": false,\n'
        '  "inference_mode": true,\n  "lora_alpha": 6.0,\n  "lora_dropout": 0.0,\n  "peft_type": "LORA",\n'
        '  "r": 3,\n  "target_modules": [\n    "q_proj",\n    "v_proj"\n  ],\n  "task_type": "CAUSAL_LM",\n'
        '  "use_dora": false,\n  "use_rslora": false\n}')
    assert json.loads(text) == cfg
    assert json.dumps(cfg, indent=2, sort_keys=True) == text  # python's pretty printer agrees here

