"""A minimal GGUF writer for tests, restated from the published GGUF layout
(the files the reference's converter writes through the `gguf` package,
utils/convert-model/src/convert_hf_safetensors_to_gguf.py:560-600):

    u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count,
    kv_count x {string key, u32 value_type, value},
    tensor_count x {string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset},
    zero padding to the alignment, then each tensor's bytes at its offset
    (offsets relative to the data section, multiples of the alignment).

Strings are {u64 length, utf-8 bytes}; arrays {u32 element_type, u64 count,
elements}.  Test infrastructure only: it writes what the tests ask, including
deliberately malformed files."""
import struct

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}

# ggml type ids and block geometry (elements, bytes) of the types the tests use
GGML = {"F32": (0, 1, 4), "F16": (1, 1, 2), "Q8_0": (8, 32, 34), "Q4_K": (12, 256, 144), "I32": (26, 1, 4),
        "BF16": (30, 1, 2)}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        body = b"".join(_str(x) if etype == STRING else struct.pack(_FMT[etype], x) for x in items)
        return struct.pack("<IQ", etype, len(items)) + body
    return struct.pack(_FMT[vtype], v)


def nbytes(type_name, ne):
    _, be, bb = GGML[type_name]
    n = 1
    for d in ne:
        n *= d
    return n // be * bb


def write_gguf(path, tensors, metadata=(), alignment=32, version=3, offsets=None, magic=MAGIC,
               truncate=None):
    """tensors: (name, type name or ggml id, ne in ggml order (innermost
    first), raw bytes).  metadata: (key, value_type, value).  A non-default
    alignment is written as general.alignment.  `offsets` overrides the
    computed data offsets; `truncate` cuts the file to that many bytes.
    Returns (data_start, offsets)."""
    kv = list(metadata)
    if alignment != 32:
        kv.append(("general.alignment", U32, alignment))
    out = struct.pack("<IIQQ", magic, version, len(tensors), len(kv))
    for key, vtype, value in kv:
        out += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
    if offsets is None:
        offsets, off = [], 0
        for _, _, _, raw in tensors:
            off = (off + alignment - 1) // alignment * alignment
            offsets.append(off)
            off += len(raw)
    for (name, gtype, ne, _), o in zip(tensors, offsets):
        gid = GGML[gtype][0] if isinstance(gtype, str) else gtype
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", gid, o)
    data_start = (len(out) + alignment - 1) // alignment * alignment
    out += b"\0" * (data_start - len(out))
    body = bytearray()
    for (_, _, _, raw), o in zip(tensors, offsets):
        if len(body) < o:
            body += b"\0" * (o - len(body))
        body[o:o + len(raw)] = raw
    out += bytes(body)
    if truncate is not None:
        out = out[:truncate]
    with open(path, "wb") as f:
        f.write(out)
    return data_start, offsets


# ---- FLUX.2 checkpoint layout ---------------------------------------------------
# The fused tensors of a diffusers FLUX.2 checkpoint and how the reference's
# loader splits them (src/ggml/GGUFLoaderVisitor.cpp:238-401): the single
# block's to_qkv_mlp_proj by rows (q | k | v | gate | up), its to_out by
# columns (attn | mlp), the feed-forward linear_in by rows (gate | up).
_ROW_FUSED = (("to_qkv_mlp_proj", ("q", "k", "v", "mlp_in_gate", "mlp_in_up")),)


def fuse_flux2(P):
    """P: parameter name -> array (PyTorch shape).  Returns file tensors
    {name: array} and, per parameter, (file tensor, "rows"|"cols", begin, end)."""
    import numpy as np
    tensors, where = {}, {}
    for name in sorted(P):
        if name in where:
            continue
        fused = None
        for mid, parts in _ROW_FUSED:
            for part in parts:
                suf = f".{mid}.{part}.weight"
                if name.endswith(suf):
                    prefix = name[: -len(suf)]
                    fused = (f"{prefix}.{mid}.weight", [f"{prefix}.{mid}.{p}.weight" for p in parts], 0)
        for part in ("attn", "mlp"):
            suf = f".to_out.{part}.weight"
            if name.endswith(suf):
                prefix = name[: -len(suf)]
                fused = (f"{prefix}.to_out.weight", [f"{prefix}.to_out.{p}.weight" for p in ("attn", "mlp")], 1)
        for part in ("gate", "up"):
            suf = f".linear_in_{part}.weight"
            if name.endswith(suf):
                prefix = name[: -len(suf)]
                fused = (f"{prefix}.linear_in.weight", [f"{prefix}.linear_in_{p}.weight" for p in ("gate", "up")], 0)
        if fused is None:
            tensors[name] = P[name]
            where[name] = (name, "rows", 0, P[name].shape[0] if P[name].ndim == 2 else 1)
            continue
        fname, members, axis = fused
        tensors[fname] = np.concatenate([P[m] for m in members], axis=axis)
        pos = 0
        for m in members:
            n = P[m].shape[axis]
            where[m] = (fname, "rows" if axis == 0 else "cols", pos, pos + n)
            pos += n
    return tensors, where


def encode(orc, a, type_name):
    """Bytes of `a` as a GGUF tensor of `type_name`, and the fp32 values a
    reader decodes from them."""
    import numpy as np
    a = np.ascontiguousarray(a, np.float32)
    if type_name == "F32":
        return a.tobytes(), a.copy()
    if type_name == "F16":
        h = a.astype(np.float16)
        return h.tobytes(), h.astype(np.float32)
    if type_name == "BF16":
        bits = orc.to_bf16_bits(a)
        return bits.tobytes(), orc.round_bf16(a)
    qt = {"Q8_0": 8, "Q4_K": 12}[type_name]
    raw = orc.quantize(a, qt)
    return raw.tobytes(), orc.dequantize(raw, a.size, qt).reshape(a.shape)


def split_like(arr, where_entry):
    """The part of file tensor `arr` a parameter takes (fuse_flux2's entry):
    rows of a matrix, elements of a vector's only row, or every row's
    columns [b, e)."""
    _, axis, b, e = where_entry
    if arr.ndim == 1:
        return arr if axis == "rows" else arr[b:e]
    return arr[b:e] if axis == "rows" else arr[:, b:e]
