"""Adapter and base-weight ingest (adapter-os_amd/host/aos_ingest.hpp, HipKernels::load_adapter*,
load_base_safetensors) through tests/cpp/aos_host_test.

The files are written here with the safetensors Python package, an implementation of the format
independent of the C++ reader. Expected adapter configs restate the rules of
MLXFFIBackend::load_adapter_with_metadata (crates/adapteros-lora-mlx-ffi/src/backend.rs:1017-1210)
as tables of cases; the first test restates the reference's own
test_load_adapter_with_metadata_overrides_inferred_defaults (backend.rs:1566-1586). Expected
float16 scales come from numpy's float32 -> float16 conversion (round to nearest even)."""
import json
import os
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import save

# AOS_HOST_TEST selects another build of the program (the sanitizer build, aos_host_test_asan)
EXE = Path(os.environ.get("AOS_HOST_TEST") or Path(__file__).resolve().parent / "cpp" / "aos_host_test")


def _exe() -> str:
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built: run make -C tests/cpp")
    return str(EXE)


def _adapter(tmp_path, tensors: dict, metadata=None, raw: bytes | None = None) -> dict:
    f = tmp_path / "adapter.safetensors"
    f.write_bytes(raw if raw is not None else save(tensors))
    cmd = [_exe(), "ingest-adapter", str(f)]
    if metadata is not None:
        cmd.append(metadata if isinstance(metadata, str) else json.dumps(metadata))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    return json.loads(r.stdout)


def _base(tmp_path, tensors: dict, key: str, raw: bytes | None = None) -> dict:
    f = tmp_path / "base.safetensors"
    f.write_bytes(raw if raw is not None else save(tensors))
    r = subprocess.run([_exe(), "ingest-base", str(f), key], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    return json.loads(r.stdout)


def _bits(a: np.ndarray) -> list[int]:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).ravel().tolist()


def _f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def _lora(modules, rank, hidden, value=1.0, fmt="prefix"):
    t = {}
    for m in modules:
        a = torch.full((rank, hidden), value, dtype=torch.float32)
        b = torch.full((hidden, rank), value, dtype=torch.float32)
        ka, kb = (f"lora_a.{m}", f"lora_b.{m}") if fmt == "prefix" else (f"{m}.lora_A", f"{m}.lora_B")
        t[ka], t[kb] = a, b
    return t


# ---- adapters ---------------------------------------------------------------------------------------


def test_reference_metadata_overrides_inferred_defaults(tmp_path):
    """backend.rs:1566-1586: q_proj and k_proj at rank 2, hidden 4; metadata rank 8, alpha 32,
    target_modules [k_proj] -> the config takes all three and only k_proj is loaded."""
    out = _adapter(tmp_path, _lora(["q_proj", "k_proj"], 2, 4),
                   {"rank": 8, "alpha": 32.0, "target_modules": ["k_proj"]})
    assert out["rank"] == 8
    assert _f32(out["alpha_bits"]) == 32.0
    assert out["target_modules"] == ["k_proj"]
    assert [m["name"] for m in out["modules"]] == ["k_proj"]
    assert _f32(out["scale_bits"]) == 4.0


def test_discovery_sorted_and_defaults(tmp_path):
    """Modules found from both key forms, sorted; no metadata -> LoRAConfig::default rank 4,
    alpha 16 (lora.rs:29-43); A/B bytes come through exactly."""
    rng = np.random.default_rng(3)
    t = {}
    data = {}
    for m, fmt in (("v_proj", "prefix"), ("q_proj", "prefix"), ("o_proj", "suffix")):
        a = rng.standard_normal((4, 64)).astype(np.float32)
        b = rng.standard_normal((32, 4)).astype(np.float32)
        data[m] = (a, b)
        ka, kb = (f"lora_a.{m}", f"lora_b.{m}") if fmt == "prefix" else (f"{m}.lora_A", f"{m}.lora_B")
        t[ka], t[kb] = torch.from_numpy(a), torch.from_numpy(b)
    t["model.norm.weight"] = torch.ones(64)
    out = _adapter(tmp_path, t)
    assert out["rank"] == 4 and _f32(out["alpha_bits"]) == 16.0 and _f32(out["scale_bits"]) == 4.0
    assert out["target_modules"] == ["o_proj", "q_proj", "v_proj"]
    assert [m["name"] for m in out["modules"]] == ["o_proj", "q_proj", "v_proj"]
    for m in out["modules"]:
        a, b = data[m["name"]]
        assert (m["rank"], m["in"], m["out"]) == (4, 64, 32)
        assert m["A"] == _bits(a) and m["B"] == _bits(b) and m["problem"] == ""


def test_no_lora_keys_gives_default_targets(tmp_path):
    out = _adapter(tmp_path, {"something.else": torch.zeros(2, 2)})
    assert out["target_modules"] == ["q_proj", "k_proj", "v_proj", "o_proj"]
    assert out["modules"] == []


def test_prefix_pair_preferred_then_suffix(tmp_path):
    """Per module the complete prefix pair wins; an incomplete prefix pair falls back to the
    suffix pair (backend.rs:1069-1088)."""
    t = {}
    t.update(_lora(["q_proj"], 2, 8, 1.0, "prefix"))
    t.update(_lora(["q_proj"], 2, 8, 2.0, "suffix"))
    t["lora_a.k_proj"] = torch.full((2, 8), 3.0)  # no lora_b.k_proj
    t.update(_lora(["k_proj"], 2, 8, 4.0, "suffix"))
    out = _adapter(tmp_path, t)
    mods = {m["name"]: m for m in out["modules"]}
    assert set(mods) == {"k_proj", "q_proj"}
    assert set(mods["q_proj"]["A"]) == {_bits(np.float32([1.0]))[0]}
    assert set(mods["k_proj"]["A"]) == {_bits(np.float32([4.0]))[0]}


RANK_CASES = [  # (metadata, rank) -- parse_rank, metadata_value_any (backend.rs:1166-1190)
    ({"rank": 8}, 8),
    ({"rank": "8"}, 8),
    ({"rank": " +12 "}, 12),
    ({"rank": 0}, 4),
    ({"rank": -3}, 4),
    ({"rank": 8.0}, 4),  # a float is no u64
    ({"rank": "8.0"}, 4),
    ({"rank": "eight"}, 4),
    ({"rank": True}, 4),
    ({"lora_rank": 12}, 12),
    ({"metadata": {"rank": 6}}, 6),
    ({"rank": 5, "metadata": {"rank": 6}}, 5),
    ({"lora_rank": 5, "metadata": {"rank": 6}}, 6),  # "rank" (top, then nested) before "lora_rank"
    ({"rank": "x", "lora_rank": 7}, 4),  # the first key found decides, even when invalid
    ({"rank": 99999999999}, 99999999999),
    ([1, 2], 4),  # not an object
]


@pytest.mark.parametrize("md,rank", RANK_CASES)
def test_metadata_rank(tmp_path, md, rank):
    assert _adapter(tmp_path, _lora(["q_proj"], 2, 4), md)["rank"] == rank


ALPHA_CASES = [  # (metadata, alpha) -- parse_alpha (backend.rs:1192-1205)
    ({"alpha": 32}, 32.0),
    ({"alpha": "0.5"}, 0.5),
    ({"alpha": " 2.5e1 "}, 25.0),
    ({"lora_alpha": 0.001}, float(np.float32(0.001))),
    ({"metadata": {"lora_alpha": "24"}}, 24.0),
    ({"alpha": "inf"}, 16.0),
    ({"alpha": -1}, 16.0),
    ({"alpha": 0}, 16.0),
    ({"alpha": "abc"}, 16.0),
    ({"alpha": "0x10"}, 16.0),
    ({"alpha": 1e39}, 16.0),  # infinite as f32
    ({"alpha": None}, 16.0),
]


@pytest.mark.parametrize("md,alpha", ALPHA_CASES)
def test_metadata_alpha(tmp_path, md, alpha):
    out = _adapter(tmp_path, _lora(["q_proj"], 2, 4), md)
    assert _f32(out["alpha_bits"]) == alpha
    assert out["scale_bits"] == _bits(np.float32([np.float32(alpha) / np.float32(out["rank"])]))[0]


TARGET_CASES = [  # (target_modules value, resulting targets) -- backend.rs:1120-1164
    (["v_proj", " q_proj ", "", "v_proj"], ["v_proj", "q_proj"]),
    (["v_proj", 3, "q_proj"], ["v_proj", "q_proj"]),
    ("q_proj, k_proj,,q_proj", ["q_proj", "k_proj"]),
    (' ["o_proj", "q_proj"] ', ["o_proj", "q_proj"]),
    ('["o_proj", 3]', None),  # not a list of strings
    ('["o_proj"', None),  # not JSON
    ([], None),
    ([1, 2], None),
    ("  ", None),
    (5, None),
    ({"q_proj": True}, None),
]


@pytest.mark.parametrize("value,targets", TARGET_CASES)
def test_metadata_target_modules(tmp_path, value, targets):
    discovered = ["k_proj", "q_proj"]
    out = _adapter(tmp_path, _lora(discovered, 2, 4), {"target_modules": value})
    want = discovered if targets is None else targets
    assert out["target_modules"] == want
    assert [m["name"] for m in out["modules"]] == [m for m in want if m in discovered]


def test_tensor_rules(tmp_path):
    """tensor_to_nested_vec (backend.rs:1371-1410): 2-D only, bytes read as float32 whatever the
    dtype; an element count that disagrees is an error."""
    t = _lora(["q_proj"], 2, 4)
    t["lora_a.q_proj"] = torch.zeros(2, 4, 1)
    out = _adapter(tmp_path, t)
    assert out["error"] == "Parse" and "Expected 2D tensor" in out["message"]
    t = _lora(["q_proj"], 2, 4)
    t["lora_b.q_proj"] = torch.zeros(4, 2, dtype=torch.float16)
    out = _adapter(tmp_path, t)
    assert out["error"] == "Parse" and "Data size mismatch" in out["message"]
    t = _lora(["q_proj"], 2, 4)
    ints = torch.arange(8, dtype=torch.int32).reshape(2, 4)
    t["lora_a.q_proj"] = ints
    out = _adapter(tmp_path, t)
    assert out["modules"][0]["A"] == ints.numpy().view(np.uint32).ravel().tolist()
    t = _lora(["q_proj"], 2, 4)
    t["lora_b.q_proj"] = torch.zeros(4, 3)
    out = _adapter(tmp_path, t)
    assert "3 columns" in out["modules"][0]["problem"]


def _lora_load(path, rank, alpha, targets) -> dict:
    r = subprocess.run([_exe(), "ingest-lora", str(path), str(rank), str(alpha), ",".join(targets)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    return json.loads(r.stdout)


def test_lora_load_with_config(tmp_path):
    """LoRAAdapter::load (lora.rs:154-216): the given config's targets only, no discovery; a target
    without weights is skipped; an unreadable path is Io, a bad file or tensor Validation."""
    f = tmp_path / "a.safetensors"
    t = _lora(["q_proj"], 2, 8, 1.0, "prefix")
    t.update(_lora(["v_proj"], 2, 8, 2.0, "suffix"))
    t.update(_lora(["k_proj"], 2, 8, 3.0, "prefix"))
    f.write_bytes(save(t))
    out = _lora_load(f, 2, 6.0, ["v_proj", "q_proj", "o_proj"])
    assert out["rank"] == 2 and _f32(out["scale_bits"]) == 3.0
    assert out["target_modules"] == ["v_proj", "q_proj", "o_proj"]
    assert [m["name"] for m in out["modules"]] == ["v_proj", "q_proj"]
    assert _lora_load(tmp_path / "missing.safetensors", 2, 6.0, ["q_proj"])["error"] == "Io"
    (tmp_path / "bad.safetensors").write_bytes(b"\x10" + bytes(7) + b"{}")
    assert _lora_load(tmp_path / "bad.safetensors", 2, 6.0, ["q_proj"])["error"] == "Validation"
    t["lora_a.q_proj"] = torch.zeros(2, 8, 1)
    f.write_bytes(save(t))
    out = _lora_load(f, 2, 6.0, ["q_proj"])
    assert out["error"] == "Validation" and "Expected 2D tensor" in out["message"]


def _raw_file(header: dict, data: bytes, header_len: int | None = None, prefix: bytes = b"") -> bytes:
    h = prefix + json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    return struct.pack("<Q", len(h) if header_len is None else header_len) + h + data


def test_safetensors_format_errors(tmp_path):
    ok = {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    assert _adapter(tmp_path, {}, raw=_raw_file(ok, bytes(8)))["modules"] == []
    bad = {
        "short": b"\x01\x02",
        "header_past_end": _raw_file(ok, bytes(8), header_len=10_000),
        "header_over_limit": struct.pack("<Q", 100_000_001) + b"{}",
        "not_brace": _raw_file(ok, bytes(8), prefix=b" "),
        "hole": _raw_file({"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, bytes(8)),
        "uncovered": _raw_file(ok, bytes(12)),
        "overlap": _raw_file({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
                              "b": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, bytes(8)),
        "size_vs_shape": _raw_file({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, bytes(8)),
        "dtype": _raw_file({"a": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 8]}}, bytes(8)),
        "json": struct.pack("<Q", 8) + b'{"a":1 }',
        "metadata_value": _raw_file({"__metadata__": {"k": 1}, **ok}, bytes(8)),
        # a shape whose element count wraps to 0 in 64 bits must not pass the size check
        "numel_overflow": _raw_file({"a": {"dtype": "F32", "shape": [2 ** 30, 2 ** 30, 16],
                                           "data_offsets": [0, 0]}}, b""),
        "dim_over_int": _raw_file({"a": {"dtype": "F32", "shape": [2 ** 32, 0], "data_offsets": [0, 0]}}, b""),
    }
    for name, raw in bad.items():
        out = _adapter(tmp_path, {}, raw=raw)
        assert out.get("error") == "Parse", (name, out)


def test_header_metadata_and_json_escapes(tmp_path):
    """__metadata__ strings and escaped tensor names (\\u escapes, surrogate pairs) parse."""
    name = "lora_a.qé\U0001F600"
    raw = save({name: torch.ones(1, 4), "lora_b.qé\U0001F600": torch.ones(4, 1)},
               metadata={"format": "pt", "note": 'a "quoted" \\ value'})
    out = _adapter(tmp_path, {}, raw=raw)
    assert out["target_modules"] == ["qé\U0001F600"]
    assert len(out["modules"]) == 1


# ---- base projections --------------------------------------------------------------------------------

F16_EDGES = np.array([0.0, -0.0, 1.0, -2.5, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf, np.nan,
                      2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -11), 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                      3 * 2.0 ** -25, 5 * 2.0 ** -25, 2.0 ** -26, 1e-10, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                      0.0999755859375, 2048.5, 4097.0], dtype=np.float32)


def _q4(out: int, inp: int, seed: int, scale_dtype, with_bias=True, scale_values=None):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 2 ** 32, size=(out, inp // 8), dtype=np.uint32)
    s = scale_values if scale_values is not None else rng.uniform(0.005, 0.03, size=(out, inp // 64))
    s = np.asarray(s, dtype=np.float32).reshape(out, inp // 64)
    b = (-8.0 * s).astype(np.float32)
    t = {"weight": torch.from_numpy(packed.view(np.int32)).view(torch.uint32)}
    t["scales"] = torch.from_numpy(s).to(scale_dtype)
    if with_bias:
        t["biases"] = torch.from_numpy(b).to(scale_dtype)
    # what the layer should receive: the stored values, as float16 bit patterns
    with np.errstate(over="ignore"):  # out-of-range values become infinities, as intended
        s16 = t["scales"].float().numpy().astype(np.float16).view(np.uint16)
        b16 = (t["biases"].float().numpy().astype(np.float16).view(np.uint16) if with_bias
               else np.zeros_like(s16))
    return t, packed, s16, b16


def _prefixed(key: str, t: dict) -> dict:
    return {f"{key}.{k}": v for k, v in t.items()}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_base_projection(tmp_path, dtype):
    t, packed, s16, b16 = _q4(64, 256, 1, dtype)
    out = _base(tmp_path, _prefixed("model.layers.0.self_attn.q_proj", t), "model.layers.0.self_attn.q_proj")
    assert out["found"] and (out["out"], out["in"]) == (64, 256)
    assert out["packed"] == packed.ravel().tolist()
    assert out["scales"] == s16.ravel().tolist() and out["biases"] == b16.ravel().tolist()


def test_base_missing_biases_are_zero_and_absent_key(tmp_path):
    t, packed, s16, _ = _q4(32, 128, 2, torch.bfloat16, with_bias=False)
    out = _base(tmp_path, _prefixed("p", t), "p")
    assert out["biases"] == [0] * (32 * 2) and out["scales"] == s16.ravel().tolist()
    assert _base(tmp_path, _prefixed("p", t), "q") == {"found": False}


def test_base_f32_to_f16_rounding(tmp_path):
    """float32 scales go to float16 bit patterns exactly as numpy rounds them (nearest even,
    overflow to infinity, subnormals)."""
    vals = np.resize(F16_EDGES, 32 * 2).reshape(32, 2)
    t, _, s16, _ = _q4(32, 128, 3, torch.float32, scale_values=vals)
    out = _base(tmp_path, _prefixed("p", t), "p")
    assert out["scales"] == s16.ravel().tolist()
    rng = np.random.default_rng(4)
    wide = (rng.standard_normal(32 * 2) * np.exp2(rng.integers(-30, 18, 32 * 2))).astype(np.float32)
    t, _, s16, b16 = _q4(32, 128, 5, torch.float32, scale_values=wide)
    out = _base(tmp_path, _prefixed("p", t), "p")
    assert out["scales"] == s16.ravel().tolist() and out["biases"] == b16.ravel().tolist()


def test_base_layout_errors(tmp_path):
    t, _, _, _ = _q4(32, 128, 6, torch.float16)
    no_scales = {k: v for k, v in t.items() if k != "scales"}
    assert _base(tmp_path, _prefixed("p", no_scales), "p")["error"] == "Validation"
    bad = dict(t)
    bad["scales"] = torch.zeros(32, 3, dtype=torch.float16)
    assert _base(tmp_path, _prefixed("p", bad), "p")["error"] == "Validation"
    bad = dict(t)
    bad["weight"] = torch.zeros(32, 16, dtype=torch.int32)
    assert _base(tmp_path, _prefixed("p", bad), "p")["error"] == "Validation"


# ---- device: file-loaded layers equal array-loaded layers bit for bit -----------------------------------


def _write_fixture(d: Path, L=2, H=256, I=512, KV=64, r1=8, r2=4, Tmax=40):
    rng = np.random.default_rng(11)
    shapes = {"q_proj": (H, H), "k_proj": (KV, H), "v_proj": (KV, H), "o_proj": (H, H),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    dtypes = [(torch.bfloat16, torch.float16), (torch.float32, torch.bfloat16)]  # (attn, mlp) per layer
    base = {}
    for l in range(L):
        for m, (o, i) in shapes.items():
            group = "self_attn" if m.endswith(("q_proj", "k_proj", "v_proj", "o_proj")) else "mlp"
            dt = dtypes[l][0 if group == "self_attn" else 1]
            t, packed, s16, b16 = _q4(o, i, 100 * l + len(base), dt, with_bias=not (l == 1 and m == "o_proj"))
            base.update(_prefixed(f"model.layers.{l}.{group}.{m}", t))
            packed.tofile(d / f"L{l}.{m}.packed.bin")
            s16.tofile(d / f"L{l}.{m}.scales.bin")
            b16.tofile(d / f"L{l}.{m}.biases.bin")
    base["model.embed_tokens.weight"] = torch.zeros(8, 8)
    (d / "base.safetensors").write_bytes(save(base, metadata={"format": "mlx"}))

    def lora(aid, names, r, fmt):
        t = {}
        for m in names:
            o, i = shapes.get(m, (64, H))
            a = (rng.standard_normal((r, i)) * 0.05).astype(np.float32)
            b = (rng.standard_normal((o, r)) * 0.05).astype(np.float32)
            if m in shapes:
                a.tofile(d / f"a{aid}.{m}.A.bin")
                b.tofile(d / f"a{aid}.{m}.B.bin")
            ka, kb = (f"lora_a.{m}", f"lora_b.{m}") if fmt == "prefix" else (f"{m}.lora_A", f"{m}.lora_B")
            t[ka], t[kb] = torch.from_numpy(a), torch.from_numpy(b)
        return t

    (d / "adapter1.safetensors").write_bytes(
        save(lora(1, ["q_proj", "v_proj", "o_proj", "gate_proj", "down_proj", "lm_head"], r1, "prefix")))
    (d / "adapter1.json").write_text(json.dumps({"metadata": {"lora_alpha": "24", "rank": r1}}))
    (d / "adapter2.safetensors").write_bytes(save(lora(2, ["k_proj", "up_proj"], r2, "suffix")))
    x = rng.standard_normal(Tmax * I).astype(np.float32)
    (x.view(np.uint32) >> 16).astype(np.uint16).tofile(d / "x.bin")
    return [str(L), str(H), str(I), str(KV), str(r1), "24", str(r2)]


def test_fixture_writer_runs_on_cpu(tmp_path):
    """The device test's fixture, parsed on the CPU: every projection is found with the
    expected float16 scales."""
    args = _write_fixture(tmp_path)
    L, H, I, KV = (int(a) for a in args[:4])
    out = _base(tmp_path, {}, "model.layers.1.self_attn.o_proj",
                raw=(tmp_path / "base.safetensors").read_bytes())
    assert out["found"] and (out["out"], out["in"]) == (H, H) and set(out["biases"]) == {0}
    assert out["scales"] == np.fromfile(tmp_path / "L1.o_proj.scales.bin", dtype=np.uint16).tolist()
    a1 = _adapter(tmp_path, {}, (tmp_path / "adapter1.json").read_text(),
                  raw=(tmp_path / "adapter1.safetensors").read_bytes())
    assert a1["rank"] == 8 and _f32(a1["scale_bits"]) == 3.0
    assert [m["name"] for m in a1["modules"]] == ["down_proj", "gate_proj", "lm_head", "o_proj", "q_proj", "v_proj"]


@pytest.mark.gpu
def test_gpu_safetensors_load_matches_array_load(tmp_path):
    """Base projections (F16, BF16 and F32 scales, one without biases) and two adapters (prefix
    keys with metadata and a module the device path skips; suffix keys without metadata) loaded
    from safetensors give the same MLP, QKV and O outputs, bit for bit, as the same weights set
    from arrays, at T = 1, 5 and 40 on both layers."""
    args = _write_fixture(tmp_path)
    r = subprocess.run([_exe(), "gpu-ingest", str(tmp_path), *args], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
