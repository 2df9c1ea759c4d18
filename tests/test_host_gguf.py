"""The GGUF checkpoint reader on the CPU, through dit_cli (no device):
`GgufInfo` reports the header, metadata and tensor table of files written by
tests/gguf_writer.py, corrupt files are rejected with a message instead of a
crash, and `Flux2Transformer2DModel --plan-only true --gguf FILE` resolves
every parameter of a small model to its file tensor, splitting the fused
tensors as the reference's GGUFLoaderVisitor does
(src/ggml/GGUFLoaderVisitor.cpp:238-401).  The oracle's Q8_0/Q4_K encoders
make the quantised payloads; the reader only sizes them here."""
import json
import os
import subprocess
import tempfile

import numpy as np
import pytest

import gguf_writer as gw
from conftest import PKG

CLI = os.path.join(PKG, "bin", "dit_cli")


def cli(*args):
    if not os.path.exists(CLI):
        pytest.skip("dit_cli not built")
    return subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=60)


def info(path):
    r = cli("GgufInfo", "--gguf", path)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.fixture
def tmp():
    with tempfile.TemporaryDirectory() as d:
        yield d


def _table(orc):
    rng = np.random.default_rng(7)
    a = rng.standard_normal((3, 64)).astype(np.float32)
    return [
        ("f32.matrix", "F32", [5, 3], rng.standard_normal(15).astype(np.float32).tobytes()),
        ("f16.vector", "F16", [7], np.arange(7, dtype=np.float16).tobytes()),
        ("bf16.cube", "BF16", [4, 3, 2], orc.to_bf16_bits(rng.standard_normal(24)).tobytes()),
        ("q8_0.weight", "Q8_0", [64, 3], orc.quantize(a, 8).tobytes()),
        ("q4_k.weight", "Q4_K", [256, 2], orc.quantize(rng.standard_normal((2, 256)), 12).tobytes()),
        ("ids", "I32", [4, 2], np.arange(8, dtype=np.int32).tobytes()),
    ]


META = [
    ("general.name", gw.STRING, "unit \"test\""),
    ("u8", gw.U8, 200), ("i8", gw.I8, -5), ("u16", gw.U16, 60000), ("i16", gw.I16, -30000),
    ("u32", gw.U32, 4000000000), ("i32", gw.I32, -2000000000), ("f32", gw.F32, 0.5), ("flag", gw.BOOL, True),
    ("u64", gw.U64, 2 ** 63 + 5), ("i64", gw.I64, -(2 ** 62)), ("f64", gw.F64, 1.25),
    ("names", gw.ARRAY, (gw.STRING, ["a", "bc", ""])), ("dims", gw.ARRAY, (gw.I32, [3, -4, 5])),
]


@pytest.mark.parametrize("alignment", [32, 64])
def test_info_reports_the_table(orc, tmp, alignment):
    tensors = _table(orc)
    path = os.path.join(tmp, "m.gguf")
    start, offs = gw.write_gguf(path, tensors, META, alignment=alignment)
    j = info(path)
    assert j["version"] == 3 and j["alignment"] == alignment and j["data_offset"] == start
    assert j["file_size"] == os.path.getsize(path)
    for (name, tname, ne, raw), off, t in zip(tensors, offs, j["tensors"]):
        assert t["name"] == name and t["type_name"] == tname and t["type"] == gw.GGML[tname][0]
        assert t["ne"] == ne and t["offset"] == start + off and t["nbytes"] == len(raw) == gw.nbytes(tname, ne)
        assert off % alignment == 0
    m = j["metadata"]
    assert m["general.name"] == 'unit "test"'
    assert (m["u8"], m["i8"], m["u16"], m["i16"]) == (200, -5, 60000, -30000)
    assert (m["u32"], m["i32"], m["flag"]) == (4000000000, -2000000000, 1)
    assert m["u64"] == 2 ** 63 + 5 and m["i64"] == -(2 ** 62)
    assert m["f32"] == 0.5 and m["f64"] == 1.25
    assert m["names"] == {"array_type": gw.STRING, "count": 3, "values": ["a", "bc", ""]}
    assert m["dims"] == {"array_type": gw.I32, "count": 3, "values": [3, -4, 5]}
    if alignment != 32:
        assert m["general.alignment"] == alignment


def test_version_2_and_directory_pick(orc, tmp):
    tensors = _table(orc)[:2]
    d = os.path.join(tmp, "ckpt")
    os.makedirs(d)
    gw.write_gguf(os.path.join(d, "b.gguf"), tensors[1:], version=3)
    gw.write_gguf(os.path.join(d, "a.gguf"), tensors, version=2)
    with open(os.path.join(d, "notes.txt"), "w") as f:
        f.write("not a checkpoint")
    j = info(d)  # a directory: its first .gguf, as the reference's loader picks one
    assert j["path"].endswith("a.gguf") and j["version"] == 2 and len(j["tensors"]) == 2


def _bad(orc, tmp, kind):
    t = _table(orc)
    path = os.path.join(tmp, kind + ".gguf")
    if kind == "magic":
        gw.write_gguf(path, t, magic=0x46554746)
    elif kind == "version":
        gw.write_gguf(path, t, version=1)
    elif kind == "truncated_header":
        start, _ = gw.write_gguf(path, t)
        with open(path, "rb") as f:
            raw = f.read()
        with open(path, "wb") as f:
            f.write(raw[: start // 2])
    elif kind == "truncated_data":
        start, offs = gw.write_gguf(path, t)
        with open(path, "rb") as f:
            raw = f.read()
        with open(path, "wb") as f:
            f.write(raw[:-5])
    elif kind == "misaligned":
        _, offs = gw.write_gguf(path, t)
        gw.write_gguf(path, t, offsets=[o + (4 if i == 2 else 0) for i, o in enumerate(offs)])
    elif kind == "unknown_type":
        gw.write_gguf(path, [("x", 99, [4], b"\0" * 16)])
    elif kind == "dims":
        gw.write_gguf(path, [("x", "F32", [1, 1, 1, 1, 2], b"\0" * 8)])
    elif kind == "duplicate":
        gw.write_gguf(path, [t[0], t[0]])
    elif kind == "alignment":
        gw.write_gguf(path, t, metadata=[("general.alignment", gw.U32, 48)])
    elif kind == "block":
        gw.write_gguf(path, [("q", "Q8_0", [48, 1], b"\0" * 34)])
    elif kind == "bytes_overflow":
        # 2^31 x 2^31 F32 elements: 2^64 bytes, which wraps to 0 in 64 bits
        gw.write_gguf(path, [("x", "F32", [2 ** 31, 2 ** 31], b"\0" * 16)])
    elif kind == "string_length":
        gw.write_gguf(path, t, metadata=[("k", gw.STRING, "v")])
        with open(path, "r+b") as f:
            f.seek(24 + 8 + 1 + 4)  # header, key length, key, type -> the value's length
            f.write((2 ** 40).to_bytes(8, "little"))
    return path


@pytest.mark.parametrize("kind,message", [
    ("magic", "bad magic"), ("version", "unsupported GGUF version 1"), ("truncated_header", "truncated"),
    ("truncated_data", "past the end of the file"), ("misaligned", "not a multiple of the alignment"),
    ("unknown_type", "unsupported ggml type 99"), ("dims", "5 dimensions"), ("duplicate", "duplicate tensor name"),
    ("alignment", "power of two"), ("block", "multiple of its block size"),
    ("string_length", "past the end of the file"), ("bytes_overflow", "more bytes than 2^64"),
])
def test_corrupt_files_are_rejected(orc, tmp, kind, message):
    r = cli("GgufInfo", "--gguf", _bad(orc, tmp, kind))
    assert r.returncode == 1, (r.returncode, r.stdout)
    assert message in r.stderr, r.stderr


SMALL = ["--num_layers", 1, "--num_single_layers", 2, "--num_attention_heads", 2, "--joint_attention_dim", 128,
         "--img_tokens", 64, "--txt_tokens", 16]
SMALL_CFG = dict(num_layers=1, num_single_layers=2, num_attention_heads=2, attention_head_dim=128,
                 in_channels=128, joint_attention_dim=128, timestep_guidance_channels=256, mlp_ratio=3.0,
                 rope_theta=2000, axes_dims_rope=[32, 32, 32, 32], eps=1e-6)


def _small_checkpoint(orc, tmp, extra=(), drop=None, reshape=None):
    import oracle.flux2 as of
    shapes = of.model_param_shapes(SMALL_CFG)
    P = {k: np.zeros(v, np.float32) for k, v in shapes.items()}
    tensors, where = gw.fuse_flux2(P)
    items = []
    for name, a in sorted(tensors.items()):
        if name == drop:
            continue
        if reshape and name == reshape:
            a = a[:-1]
        items.append((name, "F32", list(a.shape[::-1]), a.tobytes()))
    items += list(extra)
    path = os.path.join(tmp, "small.gguf")
    gw.write_gguf(path, items)
    return path, where


def test_small_model_parameters_resolve_to_fused_tensors(orc, tmp):
    """Every parameter maps to its tensor and range: direct names, the
    single blocks' to_qkv_mlp_proj rows (q | k | v | gate | up) and to_out
    columns (attn | mlp), the double block's linear_in rows (gate | up).
    A tensor no parameter takes is reported, not loaded."""
    path, where = _small_checkpoint(orc, tmp, extra=[("extra.tensor", "F32", [4], b"\0" * 16)])
    r = cli("Flux2Transformer2DModel", "--plan-only", "true", "--gguf", path, *SMALL)
    assert r.returncode == 0, r.stderr
    j = json.loads(r.stdout.strip().splitlines()[-1])
    assert j["gguf_plan"] == {k: list(v) for k, v in where.items()}
    assert j["unused"] == ["extra.tensor"]
    fused = {v[0] for v in where.values()}
    assert "single_transformer_blocks.1.attn.to_qkv_mlp_proj.weight" in fused
    assert "transformer_blocks.0.ff_context.linear_in.weight" in fused
    assert j["gguf_plan"]["single_transformer_blocks.0.attn.to_out.mlp.weight"] == [
        "single_transformer_blocks.0.attn.to_out.weight", "cols", 256, 1024]


@pytest.mark.parametrize("drop,reshape,message", [
    ("single_transformer_blocks.0.attn.to_qkv_mlp_proj.weight", None, "not found"),
    (None, "transformer_blocks.0.ff.linear_in.weight", "expected [1536, 256]"),
    (None, "proj_out.weight", "has shape [127, 256], the parameter [128, 256]"),
])
def test_missing_or_misshapen_tensors_are_named(orc, tmp, drop, reshape, message):
    path, _ = _small_checkpoint(orc, tmp, drop=drop, reshape=reshape)
    r = cli("Flux2Transformer2DModel", "--plan-only", "true", "--gguf", path, *SMALL)
    assert r.returncode == 1 and message in r.stderr, r.stderr
