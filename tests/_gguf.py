"""A minimal GGUF (version 3) writer for tests: metadata of every value type and tensors given as raw bytes, laid out as
the published GGUF specification describes (header, kv pairs, tensor infos, data aligned to general.alignment).
Written for these tests; the library's reader is the code under test."""
import struct

import numpy as np

# ggml type codes and (block elements, block bytes)
GGML = {"F32": (0, 1, 4), "F16": (1, 1, 2), "Q8_0": (8, 32, 34), "Q2_K": (10, 256, 84), "Q3_K": (11, 256, 110),
        "Q4_K": (12, 256, 144), "Q5_K": (13, 256, 176), "Q6_K": (14, 256, 210), "IQ2_XXS": (16, 256, 66)}
VT = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8, "arr": 9, "u64": 10,
      "i64": 11, "f64": 12}
PACK = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vt, v):
    if vt == 8:
        return _str(v)
    if vt == 9:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(PACK[vt], v)


def row_bytes(type_name, ne0):
    _, blk, bb = GGML[type_name]
    assert ne0 % blk == 0
    return ne0 // blk * bb


def write(path, tensors, kv=(), alignment=None, version=3, magic=b"GGUF"):
    """tensors: list of (name, type_name, ne (ggml order), raw uint8 bytes); kv: list of (key, value type, value).
    Returns {name: absolute data offset}."""
    kv = list(kv)
    align = 32
    if alignment is not None:
        kv.append(("general.alignment", "u32", alignment))
        align = alignment
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vt, v in kv:
        code = VT[vt]
        head += _str(key) + struct.pack("<I", code)
        if code == 9:
            et, items = v
            head += _value(9, (VT[et], items))
        else:
            head += _value(code, v)
    rel, offs = 0, []
    infos = b""
    for name, tn, ne, raw in tensors:
        nb = row_bytes(tn, ne[0]) * int(np.prod(ne[1:]))
        assert len(raw) == nb, (name, len(raw), nb)
        offs.append(rel)
        infos += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        infos += struct.pack("<IQ", GGML[tn][0], rel)
        rel = (rel + nb + align - 1) // align * align
    body = head + infos
    data0 = (len(body) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(body + b"\0" * (data0 - len(body)))
        for (name, tn, ne, raw), o in zip(tensors, offs):
            f.seek(data0 + o)
            f.write(np.ascontiguousarray(raw, dtype=np.uint8).tobytes())
    return {t[0]: data0 + o for t, o in zip(tensors, offs)}
