"""GPU tests of the on-disk formats (include/cfio.h and the host mirror in
cpuforge_amd.st / state / hf).

- Widening: every bf16 and f16 pattern, bitwise against the oracle's
  restatement of crates/io/src/dtype.rs (itself pinned to the reference's
  known answers and to numpy in test_oracle_io.py).
- Files: what cfio_st_write writes is byte-identical to what the
  `safetensors` crate 0.8.0 (the reference's Cargo.lock version, through its
  Python binding) serialises for the same tensors and metadata; what
  cfio_st_read_f32 reads equals the crate-written file's values, widened as
  the oracle widens them.  Small staging chunks force runs split across
  chunks and chunks holding more runs than one run table takes.
- The reference's own tests of st.rs:71-114, train/src/tests.rs:96-163
  (resume, setup mismatch, saved moments and progress) and io/src/hf.rs
  (adapter and PEFT round trips, architecture mismatch), on a small model of
  the SmolLM harness whose every op runs in libcfattn.so.
"""
import json
import os
import struct

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
safetensors = pytest.importorskip("safetensors")
from safetensors.numpy import save as np_save  # noqa: E402
from safetensors.torch import save as torch_save  # noqa: E402

DEV = "cuda"


def st():
    from cpuforge_amd import st as S
    return S


@pytest.fixture
def small_chunks():
    st().set_chunk_bytes(1 << 20)
    yield
    st().set_chunk_bytes(8 << 20)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


# ---------------------------------------------------------------- widening
@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_widen_every_pattern_bitwise(kind, offset):
    S = st()
    bits = np.arange(65536 + 13, dtype=np.uint32).astype(np.uint16)  # wraps: every pattern, ragged tail
    src = torch.from_numpy(bits.view(np.int16)).to(DEV)[offset:]
    out = torch.empty(src.numel() + 1, dtype=torch.float32, device=DEV)[offset % 2:][:src.numel()]
    fn = S.bf16_to_f32 if kind == "bf16" else S.f16_to_f32
    fn(src, out)
    want = (O.bf16_to_f32 if kind == "bf16" else O.f16_to_f32)(bits[offset:])
    assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 4099, 3_000_017])
def test_widen_sizes(n):
    S = st()
    bits = np.random.default_rng(n).integers(0, 65536, n, dtype=np.uint32).astype(np.uint16)
    src = torch.from_numpy(bits.view(np.int16)).to(DEV)
    got = host(S.f16_to_f32(src)).view(np.uint32)
    assert np.array_equal(got, O.f16_to_f32(bits).view(np.uint32))


# ---------------------------------------------------------------- files
def _tensors(seed, specs):
    rng = np.random.default_rng(seed)
    return {name: rng.standard_normal(shape).astype(np.float32) for name, shape in specs}


def _write_ours(path, arrays, meta):
    S = st()
    S.write_safetensors(path, [(n, list(a.shape), torch.from_numpy(a).to(DEV)) for n, a in arrays.items()], meta)


SPECS = [("b", (4,)), ("a", (2, 3)), ("Z", (1,)), ("scalar", ()), ("empty", (0, 7)), ("é☃\"\\\n", (5,)),
         ("big", (300, 1031)), ("model.layers.10.mlp.up_proj.lora_A", (16, 576))]


@pytest.mark.parametrize("meta", [None, {"step": "42"}, {"format": "pt"}])
def test_write_is_byte_identical_to_the_crate(tmp_path, meta):
    arrays = _tensors(1, SPECS)
    p = str(tmp_path / "ours.safetensors")
    _write_ours(p, arrays, meta)
    assert open(p, "rb").read() == np_save(arrays, metadata=meta)
    assert not os.path.exists(str(tmp_path / "ours.tmp"))


def test_write_with_several_metadata_keys(tmp_path):
    """The crate writes its metadata map in hash order; here keys are sorted.
    Everything else is byte-identical."""
    arrays = _tensors(2, SPECS)
    meta = {"step": "3", "consumed": "6", "opt_step": "3", "lora_targets": "q,v,down"}
    p = str(tmp_path / "s.safetensors")
    _write_ours(p, arrays, meta)
    ours, theirs = open(p, "rb").read(), np_save(arrays, metadata=meta)
    n1, n2 = int.from_bytes(ours[:8], "little"), int.from_bytes(theirs[:8], "little")
    assert n1 == n2 and ours[8 + n1:] == theirs[8 + n2:]
    h1, h2 = json.loads(ours[8:8 + n1]), json.loads(theirs[8:8 + n2])
    assert h1 == h2
    assert list(h1["__metadata__"]) == sorted(meta)


def test_write_many_runs_across_small_chunks(tmp_path, small_chunks):
    specs = [(f"t{i:05d}", (3,)) for i in range(9000)] + [("w", (700, 1000)), ("v", (5, 1))]
    arrays = _tensors(3, specs)
    p = str(tmp_path / "many.safetensors")
    _write_ours(p, arrays, {"k": "v"})
    assert open(p, "rb").read() == np_save(arrays, metadata={"k": "v"})


def _check_read(path, want: dict):
    S = st()
    loaded = S.read_safetensors(path)
    assert sorted(loaded.tensors) == sorted(want)
    for name, w in want.items():
        got = host(loaded.tensors[name])
        assert got.shape == w.shape, name
        assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), name
    return loaded


def test_read_f32_bf16_f16_files(tmp_path, small_chunks):
    """Runs of every dtype, odd lengths (2-byte file offsets), tensors split
    across 1 MiB chunks and more runs than one chunk's table holds."""
    rng = np.random.default_rng(4)
    ts, want = {}, {}
    shapes = [(3,), (1,), (5, 7), (), (0,), (1_000_003,), (600, 1001)] + [(1,)] * 9000
    for i, shape in enumerate(shapes):
        kind = ("f32", "bf16", "f16")[i % 3]
        n = int(np.prod(shape)) if shape else 1
        if kind == "f32":
            a = rng.standard_normal(n).astype(np.float32)
            ts[f"x{i}"] = torch.from_numpy(a).reshape(shape)
            want[f"x{i}"] = a.reshape(shape)
        else:
            bits = rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16)
            t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16 if kind == "bf16" else torch.float16)
            ts[f"x{i}"] = t.reshape(shape)
            want[f"x{i}"] = (O.bf16_to_f32 if kind == "bf16" else O.f16_to_f32)(bits).reshape(shape)
    p = str(tmp_path / "mixed.safetensors")
    with open(p, "wb") as fh:
        fh.write(torch_save(ts, metadata={"a": "1"}))
    loaded = _check_read(p, want)
    assert loaded.metadata == {"a": "1"}


def test_f32_roundtrip_with_metadata(tmp_path):
    """crates/io/src/st.rs:71-87."""
    S = st()
    p = str(tmp_path / "a.safetensors")
    a = torch.tensor([1.0, -2.5, 3.25, 0.0, 7.0, 8.0], device=DEV)
    b = torch.full((4,), 0.5, device=DEV)
    S.write_safetensors(p, [("a", [2, 3], a), ("b", [4], b)], {"step": "42"})
    ld = S.read_safetensors(p)
    assert list(ld.tensors["a"].shape) == [2, 3]
    assert host(ld.tensors["a"]).reshape(-1).tolist() == [1.0, -2.5, 3.25, 0.0, 7.0, 8.0]
    assert host(ld.tensors["b"]).tolist() == [0.5] * 4
    assert ld.metadata["step"] == "42"
    assert not (tmp_path / "a.tmp").exists()


def test_reads_bf16_and_f16_files(tmp_path):
    """crates/io/src/st.rs:89-101."""
    bf = struct.pack("<3H", 0x3F80, 0xC000, 0x4049)
    hf_ = struct.pack("<3H", 0x3C00, 0xC000, 0x7BFF)
    h = json.dumps({"bf": {"dtype": "BF16", "shape": [3], "data_offsets": [0, 6]},
                    "hf": {"dtype": "F16", "shape": [3], "data_offsets": [6, 12]}}).encode()
    p = tmp_path / "h.safetensors"
    p.write_bytes(struct.pack("<Q", len(h)) + h + bf + hf_)
    ld = st().read_safetensors(str(p))
    assert host(ld.tensors["bf"]).tolist() == [1.0, -2.0, 3.140625]
    assert host(ld.tensors["hf"]).tolist() == [1.0, -2.0, 65504.0]


def test_rejects_integer_tensors_and_missing_files(tmp_path):
    """crates/io/src/st.rs:103-113."""
    S = st()
    p = str(tmp_path / "i.safetensors")
    with open(p, "wb") as fh:
        fh.write(np_save({"ids": np.zeros(1, np.int64)}))
    with pytest.raises(S.FormatError, match="tensor 'ids' has unsupported dtype I64"):
        S.read_safetensors(p)
    with pytest.raises(S.FormatError):
        S.read_safetensors(str(tmp_path / "nope"))


def test_write_errors(tmp_path):
    S = st()
    x = torch.zeros(3, device=DEV)
    with pytest.raises(S.FormatError, match="cannot write"):
        S.write_safetensors(str(tmp_path / "no" / "such" / "dir.safetensors"), [("x", [3], x)])
    with pytest.raises(S.FormatError, match="duplicate tensor name"):
        S.write_safetensors(str(tmp_path / "d.safetensors"), [("x", [3], x), ("x", [3], x)])


def test_read_is_ordered_on_the_stream_after_close(tmp_path):
    """The call returns once the bytes are staged: the file can be closed and
    the next kernel on the stream sees the data."""
    S = st()
    a = np.random.default_rng(5).standard_normal(5_000_000).astype(np.float32)
    p = str(tmp_path / "big.safetensors")
    with open(p, "wb") as fh:
        fh.write(np_save({"a": a}))
    out = torch.empty(a.size, dtype=torch.float32, device=DEV)
    from cpuforge_amd.attention import default_context
    with S.StFile(p) as f:
        f.read([0], [out], default_context())
    s = (out * 2.0).sum()
    assert abs(float(s) - float(a.astype(np.float64).sum() * 2.0)) < 1e-2 * np.sqrt(a.size)
    assert np.array_equal(host(out), a)


# ---------------------------------------------------------------- training state and adapters
CFG = dict(vocab=96, d=128, ffn=96, heads=4, kv_heads=2, head_dim=64, eps=1e-5, theta=1e4)
SEQ = 64


def mk(seed, train="lora", config=None):
    from cpuforge_amd.train_bench import SmolLM
    return SmolLM(layers=2, seq=SEQ, rank=0, seed=seed, config=config or CFG, train=train)


def batches(n, seed=11, batch=2):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    out = []
    for _ in range(n):
        t = torch.randint(0, CFG["vocab"], (batch, SEQ), generator=g, device=DEV)
        y = torch.randint(0, CFG["vocab"], (batch, SEQ), generator=g, device=DEV)
        out.append((t, y))
    return out


def opt():
    from cpuforge_amd.optim import AdamW
    return AdamW(0.9, 0.999, 1e-8, 0.01)


def run(model, o, data, lr=1e-2):
    losses = []
    for tokens, targets in data:
        for p in model.params():
            p.grad = None
        loss = model.loss(tokens, targets)
        loss.backward()
        o.update(model, lr)
        losses.append(loss.item())
    return losses


def test_resume_continues_exactly_where_it_stopped(tmp_path):
    """crates/train/src/tests.rs:96-133."""
    from cpuforge_amd.state import load_state, save_state
    data = batches(8)
    path = str(tmp_path / "state.safetensors")

    def mk_lora():
        m = mk(4)
        m.add_lora(4, 8.0, ["q", "v", "down"], 9)
        return m

    straight, o1 = mk_lora(), opt()
    straight_losses = run(straight, o1, data)

    first, o2 = mk_lora(), opt()
    run(first, o2, data[:4])
    save_state(path, first, o2, 4, 8)

    second, o3 = mk(4), opt()  # same base weights, no adapter yet
    second.add_lora(4, 8.0, ["q", "v", "down"], 123)
    step, consumed = load_state(path, second, o3)
    assert (step, consumed) == (4, 8) and o3.step == 4
    resumed = run(second, o3, data[4:])
    assert len(resumed) == 4
    for x, y in zip(straight_losses[4:], resumed):
        assert abs(x - y) < 1e-5, (x, y)
    worst = max(float((a - b).detach().abs().max())
                for (_, a), (_, b) in zip(straight.named_params(), second.named_params()))
    assert worst < 1e-5, worst


def test_resume_attaches_the_files_adapters_to_a_plain_model(tmp_path):
    """state.rs:65-75: a model without adapters gets the file's (rank,
    alpha, targets) attached before the tensors are restored."""
    from cpuforge_amd.state import load_state, save_state
    m = mk(6)
    m.add_lora(4, 8.0, ["q", "up"], 3)
    o = opt()
    run(m, o, batches(2))
    path = str(tmp_path / "s.safetensors")
    save_state(path, m, o, 2, 4)
    fresh, o2 = mk(6), opt()
    assert load_state(path, fresh, o2) == (2, 4)
    assert fresh.lora_cfg == m.lora_cfg
    for (n1, a), (n2, b) in zip(m.named_params(), fresh.named_params()):
        assert n1 == n2 and torch.equal(a, b), n1
    assert sorted(o2.state) == sorted(o.state)
    for k in o.state:
        assert torch.equal(o.state[k][0], o2.state[k][0]) and torch.equal(o.state[k][1], o2.state[k][1])


def test_resume_rejects_a_state_from_a_different_setup(tmp_path):
    """crates/train/src/tests.rs:135-149."""
    from cpuforge_amd.st import FormatError
    from cpuforge_amd.state import load_state, save_state
    m = mk(5)
    m.add_lora(4, 8.0, ["q"], 1)
    o = opt()
    run(m, o, batches(2))
    path = str(tmp_path / "s.safetensors")
    save_state(path, m, o, 2, 4)
    other = mk(5)
    other.add_lora(8, 8.0, ["q"], 1)
    with pytest.raises(FormatError, match="differs"):
        load_state(path, other, opt())


def test_saved_state_includes_optimizer_moments_and_progress(tmp_path):
    """crates/train/src/tests.rs:151-163 (full training: every parameter
    has p / m / v)."""
    from cpuforge_amd.state import save_state
    m, o = mk(6, train="full"), opt()
    run(m, o, batches(3))
    path = str(tmp_path / "s.safetensors")
    save_state(path, m, o, 3, 6)
    ld = st().read_safetensors(path)
    assert ld.metadata["step"] == "3" and ld.metadata["consumed"] == "6" and ld.metadata["opt_step"] == "3"
    for k in ("p.model.embed_tokens.weight", "m.model.layers.0.mlp.up_proj.weight", "v.model.norm.weight"):
        assert k in ld.tensors
    assert torch.equal(ld.tensors["p.model.norm.weight"], m.final_norm)
    assert torch.equal(ld.tensors["m.model.norm.weight"], o.state["model.norm.weight"][0])
    n = sum(1 for _ in m.named_params())
    assert len(ld.tensors) == 3 * n


def _lora_model(seed, rank=3, alpha=6.0, targets=("q", "v", "down")):
    m = mk(seed)
    m.add_lora(rank, alpha, list(targets), 7)
    g = torch.Generator(device=DEV)
    g.manual_seed(8)
    with torch.no_grad():
        for layer in m.layers:
            for attr in ("wq", "wv", "down"):
                lin = layer[attr]
                if lin.b is not None:
                    lin.b.copy_(torch.randn(lin.b.shape, generator=g, device=DEV) * 0.3)
    return m


def _loss(m):
    t, y = batches(1, seed=99)[0]
    with torch.no_grad():
        return float(m.loss(t, y))


def test_adapter_roundtrip_restores_behaviour(tmp_path):
    """crates/io/src/hf.rs:242-265."""
    from cpuforge_amd.hf import load_adapter, save_adapter
    base = _lora_model(4)
    want = _loss(base)
    path = str(tmp_path / "adapter.safetensors")
    save_adapter(path, base)
    fresh = mk(4)
    assert _loss(fresh) != want
    load_adapter(fresh, path)
    assert _loss(fresh) == want
    assert fresh.lora_cfg == base.lora_cfg


def test_peft_adapter_roundtrips_with_peft_names_and_config(tmp_path):
    """crates/io/src/hf.rs:267-297."""
    from cpuforge_amd.hf import load_peft_adapter, save_peft_adapter
    from cpuforge_amd.st import FormatError, StFile
    base = _lora_model(4)
    want = _loss(base)
    d = str(tmp_path)
    save_peft_adapter(d, base, "org/base")
    c = json.loads(open(os.path.join(d, "adapter_config.json")).read())
    assert (c["peft_type"], c["r"], c["lora_alpha"]) == ("LORA", 3, 6.0)
    assert c["base_model_name_or_path"] == "org/base"
    assert c["target_modules"] == ["q_proj", "v_proj", "down_proj"]
    with StFile(os.path.join(d, "adapter_model.safetensors")) as f:
        names = [n for n, _, _, _ in f.tensors()]
        assert f.metadata() == {"format": "pt"}
    assert "base_model.model.model.layers.0.self_attn.q_proj.lora_A.weight" in names
    assert "base_model.model.model.layers.1.mlp.down_proj.lora_B.weight" in names
    assert len(names) == 2 * 3 * 2
    fresh = mk(4)
    load_peft_adapter(fresh, d)
    assert _loss(fresh) == want
    with open(os.path.join(d, "adapter_config.json"), "w") as fh:
        fh.write(json.dumps(c).replace("LORA", "IA3"))
    with pytest.raises(FormatError):
        load_peft_adapter(mk(4), d)


def test_adapter_for_a_different_architecture_is_rejected(tmp_path):
    """crates/io/src/hf.rs:318-343."""
    from cpuforge_amd.hf import load_adapter, save_adapter
    from cpuforge_amd.st import FormatError
    a = mk(5)
    a.add_lora(2, 4.0, ["q"], 1)
    path = str(tmp_path / "a.safetensors")
    save_adapter(path, a)
    wide = mk(6, config=dict(CFG, d=256))
    with pytest.raises(FormatError, match="shape"):
        load_adapter(wide, path)
    with pytest.raises(FormatError):
        save_adapter(path, mk(7))


def test_state_file_is_what_the_crate_writes(tmp_path):
    """save_state's file, tensor for tensor and byte for byte in the data
    section, equals the crate's serialisation of the same host arrays."""
    from cpuforge_amd.state import save_state
    m = mk(8)
    m.add_lora(4, 8.0, ["q", "k", "v", "o", "gate", "up", "down"], 2)
    o = opt()
    run(m, o, batches(1))
    path = str(tmp_path / "s.safetensors")
    save_state(path, m, o, 1, 2)
    arrays = {}
    for name, p in m.named_params():
        if p.requires_grad:
            arrays[f"p.{name}"] = host(p)
            arrays[f"m.{name}"] = host(o.state[name][0])
            arrays[f"v.{name}"] = host(o.state[name][1])
    meta = {"step": "1", "consumed": "2", "opt_step": "1", "lora_rank": "4", "lora_alpha": "8",
            "lora_targets": "q,k,v,o,gate,up,down"}
    ours, theirs = open(path, "rb").read(), np_save(arrays, metadata=meta)
    n1, n2 = int.from_bytes(ours[:8], "little"), int.from_bytes(theirs[:8], "little")
    assert json.loads(ours[8:8 + n1]) == json.loads(theirs[8:8 + n2])
    assert ours[8 + n1:] == theirs[8 + n2:]
