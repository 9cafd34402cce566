"""Checkpoint ingest on the CPU: the memory-mapped safetensors reader against files
written by the `safetensors` package (the format's own implementation) and by a
writer that follows the reference's write_mock_safetensors
(crates/objeta-cuda/src/bin/deepseek_single_layer_moe.rs:2685-2740), and the
DeepSeek lookups against the behaviour the reference's own tests assert
(test_missing_router_fails_clearly, test_missing_expert_tensor_fails_clearly,
test_missing_scale_tensor_fails, test_router_shape_mismatch_fails,
test_block_family_distinction, deepseek_single_layer_moe.rs:3117-4040)."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from objeta_amd import HipError
from objeta_amd.safetensors import ModelWeights


def write_mock(path, tensors, metadata=None, pad=True):
    """tensors: {name: (dtype, shape, bytes)} laid out in insertion order; the header
    padded so the data starts 8-byte aligned, as the reference's mock writer does."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, data) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    if metadata is not None:
        header["__metadata__"] = metadata
    js = json.dumps(header).encode()
    if pad:
        js += b" " * ((8 - len(js) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)))
        f.write(js)
        for b in blobs:
            f.write(b)


def test_reads_files_written_by_the_safetensors_package(tmp_path):
    g = torch.Generator().manual_seed(3)
    ts = {
        "a.f32": torch.randn(3, 5, generator=g),
        "b.f16": torch.randn(7, generator=g).half(),
        "c.bf16": torch.randn(2, 4, generator=g).bfloat16(),
        "d.i8": torch.randint(-128, 127, (16,), dtype=torch.int8, generator=g),
        "e.u8": torch.randint(0, 255, (4, 4), dtype=torch.uint8, generator=g),
        "f.i64": torch.arange(5, dtype=torch.int64),
        "g.f8": torch.randn(8, 16, generator=g).to(torch.float8_e4m3fn),
        "h.scalar": torch.tensor(2.5),
    }
    p = tmp_path / "m.safetensors"
    save_file(ts, str(p), metadata={"format": "pt"})
    m = ModelWeights(p)
    assert len(m) == len(ts) and m.keys() == sorted(ts)
    for name, t in ts.items():
        info = m.info(name)
        assert info.shape == tuple(t.shape) and info.nbytes == t.numel() * t.element_size()
        raw = t.contiguous().view(torch.uint8).numpy().tobytes() if t.dim() else t.reshape(1).view(torch.uint8).numpy().tobytes()
        assert m.get_raw(name).tobytes() == raw
    assert {n: m.info(n).dtype for n in ts} == {"a.f32": "F32", "b.f16": "F16", "c.bf16": "BF16", "d.i8": "I8",
                                              "e.u8": "U8", "f.i64": "I64", "g.f8": "F8_E4M3", "h.scalar": "F32"}
    assert np.array_equal(m.get_f32("a.f32"), ts["a.f32"].numpy().ravel())
    assert np.array_equal(m.get_f32("b.f16"), ts["b.f16"].float().numpy())
    assert np.array_equal(m.get_f32("c.bf16"), ts["c.bf16"].float().numpy().ravel())
    r, c, mat = m.get_matrix("a.f32")
    assert (r, c) == (3, 5) and np.array_equal(mat, ts["a.f32"].numpy())
    with pytest.raises(HipError) as e:
        m.get_f32("d.i8")
    assert "cannot convert I8 to f32" in str(e.value)
    with pytest.raises(HipError) as e:
        m.get_raw("nope")
    assert e.value.status == 4 and "missing tensor: nope" in str(e.value)  # OBJETA_HIP_ERR_IO
    assert m.info("nope") is None and not m.contains("nope") and m.contains("a.f32")
    m.close()


def test_f16_conversion_matches_ieee_on_every_pattern(tmp_path):
    """half_to_f32 (lib.rs:297-323): exact on every pattern; NaN payloads become the
    canonical NaN, as f32::NAN."""
    bits = np.arange(65536, dtype=np.uint16)
    write_mock(tmp_path / "h.safetensors", {"h": ("F16", [65536], bits.tobytes()),
                                            "b": ("BF16", [65536], bits.tobytes())})
    m = ModelWeights(tmp_path / "h.safetensors")
    got = m.get_f32("h")
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert (got[nan].view(np.uint32) == 0x7FC00000).all()
    assert np.array_equal(m.get_f32("b").view(np.uint32), bits.astype(np.uint32) << 16)


def test_shards_in_name_order_and_replacement(tmp_path):
    d = tmp_path / "model"
    d.mkdir()
    write_mock(d / "model-00002-of-00002.safetensors", {"x": ("U8", [2], b"\x02\x02"), "z": ("U8", [1], b"\x09")})
    write_mock(d / "model-00001-of-00002.safetensors", {"x": ("U8", [2], b"\x01\x01"), "y": ("U8", [1], b"\x07")})
    (d / "notes.txt").write_text("ignored")
    m = ModelWeights(d)
    assert m.keys() == ["x", "y", "z"]
    assert m.get_raw("x").tobytes() == b"\x02\x02" and m.info("x").file == 1  # the later shard wins
    assert m.get_raw("y").tobytes() == b"\x07" and m.info("y").file == 0


def test_header_names_with_escapes_and_metadata(tmp_path):
    p = tmp_path / "e.safetensors"
    write_mock(p, {"café.\U0001F600.w": ("U8", [1], b"\x05"), 'q"uote\\s': ("U8", [1], b"\x06")},
               metadata={"k": "v"}, pad=False)
    m = ModelWeights(p)
    assert sorted(m.keys()) == sorted(["café.\U0001F600.w", 'q"uote\\s'])
    assert m.get_raw("café.\U0001F600.w").tobytes() == b"\x05"


@pytest.mark.parametrize("case", ["short", "header_len", "json", "dtype", "offsets", "entry", "utf8"])
def test_malformed_files_fail_with_io_errors(tmp_path, case):
    p = tmp_path / "bad.safetensors"
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "header_len":
        p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    elif case == "json":
        js = b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]'
        p.write_bytes(struct.pack("<Q", len(js)) + js + b"\x00")
    elif case == "dtype":
        write_mock(p, {"a": ("F12", [1], b"\x00")})
    elif case == "offsets":
        js = json.dumps({"a": {"dtype": "U8", "shape": [8], "data_offsets": [0, 8]}}).encode()
        p.write_bytes(struct.pack("<Q", len(js)) + js + b"\x00" * 4)
    elif case == "entry":
        js = json.dumps({"a": {"dtype": "U8", "shape": [1]}}).encode()
        p.write_bytes(struct.pack("<Q", len(js)) + js + b"\x00")
    else:
        js = b'{"\xff": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}'
        p.write_bytes(struct.pack("<Q", len(js)) + js + b"\x00")
    with pytest.raises(HipError) as e:
        ModelWeights(p)
    assert e.value.status == 4, str(e.value)
    msg = str(e.value)
    want = {"short": "file too short", "header_len": "header length exceeds file size", "json": "invalid header JSON",
            "dtype": "Unknown dtype: F12", "offsets": "outside the file", "entry": "invalid tensor entry for 'a'",
            "utf8": "invalid UTF-8"}[case]
    assert want in msg, msg


# ------------------------------------------------------------------ DeepSeek naming
def fp4_tensors(prefix, rows, cols, rng):
    w = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    s = rng.integers(119, 128, rows * cols // 32, dtype=np.uint8)
    return {f"{prefix}.weight": ("I8", [rows, cols // 2], w.tobytes()),
            f"{prefix}.scale": ("F8_E8M0", [rows, cols // 32], s.tobytes())}


def fp8_tensors(prefix, rows, cols, rng):
    w = rng.integers(0, 256, rows * cols, dtype=np.uint8)
    s = rng.integers(119, 128, ((rows + 127) // 128) * ((cols + 127) // 128), dtype=np.uint8)
    return {f"{prefix}.weight": ("F8_E4M3", [rows, cols], w.tobytes()),
            f"{prefix}.scale": ("F8_E8M0", [(rows + 127) // 128, (cols + 127) // 128], s.tobytes())}


def deepseek_checkpoint(path, hidden=256, inter=128, experts=3, layers=(0, 1), mtp=True, seed=0):
    rng = np.random.default_rng(seed)
    t = {}
    fams = ["layers"] + (["mtp"] if mtp else [])
    for fam in fams:
        for l in layers:
            base = f"{fam}.{l}.ffn"
            for e in range(experts):
                t.update(fp4_tensors(f"{base}.experts.{e}.w1", inter, hidden, rng))
                t.update(fp4_tensors(f"{base}.experts.{e}.w3", inter, hidden, rng))
                t.update(fp4_tensors(f"{base}.experts.{e}.w2", hidden, inter, rng))
            t.update(fp8_tensors(f"{base}.shared_experts.w1", inter, hidden, rng))
            t.update(fp8_tensors(f"{base}.shared_experts.w3", inter, hidden, rng))
            t.update(fp8_tensors(f"{base}.shared_experts.w2", hidden, inter, rng))
            router = torch.randn(experts, hidden, generator=torch.Generator().manual_seed(l)).bfloat16()
            t[f"{base}.gate.weight"] = ("BF16", [experts, hidden], router.view(torch.uint16).numpy().tobytes())
            t[f"{base}.gate.tid2eid"] = ("I32", [4], np.arange(4, dtype=np.int32).tobytes())
            t[f"{fam}.{l}.hc_ffn_base"] = ("F32", [4], np.zeros(4, np.float32).tobytes())
    write_mock(path, t)
    return t


def test_deepseek_routed_expert_lookup(tmp_path):
    p = tmp_path / "ds.safetensors"
    t = deepseek_checkpoint(p)
    m = ModelWeights(p)
    for fam, mtp in (("layers", False), ("mtp", True)):
        for l in (0, 1):
            for e in range(3):
                parts, dims = m.deepseek_expert(l, e, mtp)
                assert dims == (256, 128, 256)
                names = [f"{fam}.{l}.ffn.experts.{e}.{w}.{k}" for w in ("w1", "w3", "w2") for k in ("weight", "scale")]
                for arr, n in zip(parts, names):
                    assert arr.tobytes() == t[n][2], n


def test_deepseek_shared_expert_and_router(tmp_path):
    p = tmp_path / "ds.safetensors"
    t = deepseek_checkpoint(p)
    m = ModelWeights(p)
    parts, dims = m.deepseek_shared_expert(1)
    assert dims == (256, 128, 256)
    names = [f"layers.1.ffn.shared_experts.{w}.{k}" for w in ("w1", "w3", "w2") for k in ("weight", "scale")]
    assert all(a.tobytes() == t[n][2] for a, n in zip(parts, names))
    # test_block_family_distinction (deepseek_single_layer_moe.rs:3973-4040)
    name, w = m.deepseek_router(0)
    assert name == "layers.0.ffn.gate.weight" and w.shape == (3, 256)
    want = np.frombuffer(t[name][2], np.uint16).astype(np.uint32) << 16
    assert np.array_equal(w.ravel().view(np.uint32), want)
    assert m.deepseek_router(0, mtp=True)[0] == "mtp.0.ffn.gate.weight"


def test_deepseek_lookup_errors_follow_the_reference(tmp_path):
    p = tmp_path / "ds.safetensors"
    t = deepseek_checkpoint(p, layers=(0,), mtp=False)
    m = ModelWeights(p)
    # test_missing_expert_tensor_fails_clearly: every kind missing for an absent expert
    with pytest.raises(HipError) as e:
        m.deepseek_expert(0, 7)
    assert 'layer 0 block family Decoder expert 7 missing tensors: ["gate", "up", "down"]' in str(e.value)
    # test_missing_router_fails_clearly
    with pytest.raises(HipError) as e:
        m.deepseek_router(5)
    assert "no router tensor found for layer 5 and block family Decoder" in str(e.value)
    # a shared expert of a missing layer: the Io error of get_raw
    with pytest.raises(HipError) as e:
        m.deepseek_shared_expert(3)
    assert e.value.status == 4 and "layers.3.ffn.shared_experts.w1.weight" in str(e.value)
    # test_missing_scale_tensor_fails
    t2 = {k: v for k, v in t.items() if k != "layers.0.ffn.experts.1.w3.scale"}
    write_mock(tmp_path / "noscale.safetensors", t2)
    with pytest.raises(HipError) as e:
        ModelWeights(tmp_path / "noscale.safetensors").deepseek_expert(0, 1)
    assert "has no scale tensor" in str(e.value)
    # test_router_shape_mismatch_fails: a 1-D router tensor
    t3 = dict(t)
    t3["layers.0.ffn.gate.weight"] = ("BF16", [3 * 256], t["layers.0.ffn.gate.weight"][2])
    write_mock(tmp_path / "r1d.safetensors", t3)
    with pytest.raises(HipError) as e:
        ModelWeights(tmp_path / "r1d.safetensors").deepseek_router(0)
    assert "expected [num_experts, hidden_size]" in str(e.value)
    # two gate.weight tensors for one layer are ambiguous
    t4 = dict(t)
    t4["layers.0.mlp.gate.weight"] = t["layers.0.ffn.gate.weight"]
    write_mock(tmp_path / "amb.safetensors", t4)
    with pytest.raises(HipError) as e:
        ModelWeights(tmp_path / "amb.safetensors").deepseek_router(0)
    assert "2 router tensors found for layer 0" in str(e.value)
    # a weight with the wrong shape for its scale
    t5 = dict(t)
    t5["layers.0.ffn.experts.0.w1.scale"] = ("F8_E8M0", [128, 4], t["layers.0.ffn.experts.0.w1.scale"][2][:512])
    write_mock(tmp_path / "shape.safetensors", t5)
    with pytest.raises(HipError) as e:
        ModelWeights(tmp_path / "shape.safetensors").deepseek_expert(0, 0)
    assert "gate scale" in str(e.value)


@pytest.mark.parametrize("name,kind", [("layers.0.ffn.experts.1.w2.weight", "routed"),
                                       ("layers.0.ffn.experts.2.w1.scale", "routed"),
                                       ("layers.0.ffn.shared_experts.w3.weight", "shared"),
                                       ("layers.0.ffn.shared_experts.w2.scale", "shared")])
def test_truncated_expert_tensor_fails_before_use(tmp_path, name, kind):
    """A tensor whose data holds fewer bytes than its shape has one-byte elements (a
    truncated checkpoint) is rejected by the expert lookups, so no kernel is handed a
    block shorter than the shape it reads."""
    t = deepseek_checkpoint(tmp_path / "ok.safetensors", layers=(0,), mtp=False)
    dtype, shape, data = t[name]
    t[name] = (dtype, shape, data[:-1])
    write_mock(tmp_path / "trunc.safetensors", t)
    m = ModelWeights(tmp_path / "trunc.safetensors")
    with pytest.raises(HipError) as e:
        if kind == "routed":
            m.deepseek_expert(0, int(name.split(".")[4]))
        else:
            m.deepseek_shared_expert(0)
    assert e.value.status == 5 and "one-byte elements" in str(e.value)  # OBJETA_HIP_ERR_INVALID_INPUT
    assert f"{len(data) - 1} bytes for {len(data)}" in str(e.value)


def test_views_keep_the_mapping_alive(tmp_path):
    p = tmp_path / "ds.safetensors"
    t = deepseek_checkpoint(p, layers=(0,), mtp=False)
    parts, _ = ModelWeights(p).deepseek_expert(0, 2)  # the model object itself is dropped at once
    import gc
    gc.collect()
    assert parts[0].tobytes() == t["layers.0.ffn.experts.2.w1.weight"][2]
