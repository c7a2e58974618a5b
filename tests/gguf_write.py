"""A minimal GGUF writer for the tests (little-endian, v3 by default).

Builds files byte by byte from the GGUF layout, so the reader is checked
against bytes it did not produce itself.
"""

import struct

_CODES = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}


def _str(s):
    b = s.encode("utf-8", "surrogateescape") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype in _CODES:
        return struct.pack("<" + _CODES[vtype], v)
    if vtype == 8:
        return _str(v)
    if vtype == 9:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    raise ValueError(vtype)


def gguf_bytes(kv, tensors, alignment=32, version=3, magic=b"GGUF", offsets=None):
    """kv: [(key, vtype, value)]; tensors: [(name, ggml_type, ne, raw bytes)].

    `offsets` overrides a tensor's relative data offset by name (for malformed
    files)."""
    kv = list(kv)
    if alignment != 32:
        kv.append(("general.alignment", 4, alignment))
    head = bytearray(magic) + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vtype, v in kv:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    data = bytearray()
    for name, gtype, ne, raw in tensors:
        data += b"\0" * (-len(data) % alignment)
        rel = (offsets or {}).get(name, len(data))
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", gtype, rel)
        data += raw
    head += b"\0" * (-len(head) % alignment)
    return bytes(head + data)


def write(path, kv, tensors, **kw):
    with open(path, "wb") as fh:
        fh.write(gguf_bytes(kv, tensors, **kw))
    return path
