"""Minimal GGUF tensor-table reader for tests (header layout as in
core/gguf_parser.cpp:164-324): returns {name: (type, shape, absolute offset)}."""
import struct

_SIZES = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def _skip(f, kind):
    if kind == 8:
        (n,) = struct.unpack("<Q", f.read(8))
        f.seek(n, 1)
    elif kind == 9:
        at, n = struct.unpack("<IQ", f.read(12))
        for _ in range(n):
            _skip(f, at)
    else:
        f.seek(_SIZES[kind], 1)


def tensors(path, honour_alignment=True):
    """general.alignment (a u32) sets the data section's alignment as the GGUF
    format defines; the reference ignores the key and uses 32
    (core/gguf_parser.cpp:30, 196): honour_alignment=False reads as it does."""
    align = 32
    with open(path, "rb") as f:
        assert f.read(4) == b"GGUF"
        _, nt, nkv = struct.unpack("<IQQ", f.read(20))
        for _ in range(nkv):
            (n,) = struct.unpack("<Q", f.read(8))
            key = f.read(n).decode()
            (kind,) = struct.unpack("<I", f.read(4))
            if key == "general.alignment" and kind == 4 and honour_alignment:
                (align,) = struct.unpack("<I", f.read(4))
            else:
                _skip(f, kind)
        out = {}
        for _ in range(nt):
            (n,) = struct.unpack("<Q", f.read(8))
            name = f.read(n).decode()
            (nd,) = struct.unpack("<I", f.read(4))
            shape = struct.unpack(f"<{nd}Q", f.read(8 * nd))
            t, off = struct.unpack("<IQ", f.read(12))
            out[name] = (t, shape, off)
        data = (f.tell() + align - 1) // align * align
    return {k: (t, s, data + o) for k, (t, s, o) in out.items()}
