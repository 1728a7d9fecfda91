"""GGUF files: the reader is the library's parser (bb_gguf_*, mirroring GgufFile in gguf.rs and
config::validate in config.rs:51-89); the writer serialises metadata and tensors in the same
container format (version 3, little-endian, tensor data aligned) for synthetic model files.

Reader names follow gguf.rs: GgufFile.open / from_bytes, .version, .alignment, .data_offset,
.tensors (TensorInfo), tensor_data, get / get_u32 / get_f32 / get_str / get_u32_array /
get_str_array, architecture(). Accessors return None where the reference's return None.
"""
import ctypes
import struct
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import BBError, check, lib

# Metadata value types (gguf.rs:61-75).
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}


@dataclass
class TensorInfo:
    """TensorInfo (gguf.rs:123-140)."""
    name: str
    dims: list
    ggml_type: int
    offset: int
    data_start: int
    data_len: int
    index: int

    def n_elements(self):
        n = 1
        for d in self.dims:
            n *= d
        return n


def _missing(rc):
    if rc == _lib.BB_ERR_MISSING:
        return True
    check(rc)
    return False


class _Mapping:
    """Owner of a parsed file's native handle (its mapping or byte copy): closed when the last
    reference goes, so the GgufFile and every zero-copy tensor view keep it alive."""

    def __init__(self, handle):
        self.handle = handle

    def __del__(self):
        h, self.handle = self.handle, None
        if h:
            try:
                lib().bb_gguf_close(h)
            except Exception:
                pass


class GgufFile:
    """A parsed GGUF file (gguf.rs:143-275): a read-only mapping of the file, or a copy of bytes."""

    def __init__(self, handle):
        self._map = _Mapping(handle)
        v, a, d = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
        nt, nm = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().bb_gguf_header(handle, ctypes.byref(v), ctypes.byref(a), ctypes.byref(d), ctypes.byref(nt),
                                   ctypes.byref(nm)))
        self.version, self.alignment, self.data_offset = v.value, a.value, d.value
        self.tensors = []
        info = _lib.GgufTensorInfo()
        for i in range(nt.value):
            check(lib().bb_gguf_tensor(handle, i, ctypes.byref(info)))
            self.tensors.append(TensorInfo(info.name.decode(), [info.dims[k] for k in range(info.n_dims)],
                                           info.ggml_type, info.offset, info.data_start, info.data_len, i))
        self.keys = []
        key = ctypes.c_char_p()
        for i in range(nm.value):
            check(lib().bb_gguf_meta_key(handle, i, ctypes.byref(key)))
            self.keys.append(key.value.decode())

    @classmethod
    def open(cls, path):
        h = ctypes.c_void_p()
        check(lib().bb_gguf_open(str(path).encode(), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def from_bytes(cls, data):
        buf = bytes(data)
        h = ctypes.c_void_p()
        check(lib().bb_gguf_open_bytes(buf, len(buf), ctypes.byref(h)))
        return cls(h)

    @property
    def handle(self):
        m = getattr(self, "_map", None)
        return m.handle if m is not None else None

    def close(self):
        """Ends this object's use of the file; the mapping itself is released once no tensor
        view returned by tensor_data is alive any more."""
        self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, name):
        """Model::tensor (model.rs:80-82): the TensorInfo of `name`, or None."""
        i = ctypes.c_size_t()
        if _missing(lib().bb_gguf_find_tensor(self.handle, name.encode(), ctypes.byref(i))):
            return None
        return self.tensors[i.value]

    def tensor_data(self, t):
        """tensor_data (gguf.rs:191-193): a zero-copy uint8 view of the tensor's bytes. The view
        holds the file's mapping (as the reference's slice borrows the GgufFile), so it stays
        valid after close() or after the GgufFile itself is gone."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        check(lib().bb_gguf_tensor_data(self.handle, t.index, ctypes.byref(p), ctypes.byref(n)))
        if n.value == 0:
            return np.zeros(0, np.uint8)
        buf = (ctypes.c_uint8 * n.value).from_address(p.value)
        buf._owner = self._map  # the numpy array's base is buf
        return np.ctypeslib.as_array(buf)

    def meta_type(self, key):
        """(value type, element type, items) of a key, or None when absent."""
        vt, et, n = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_size_t()
        if _missing(lib().bb_gguf_meta_type(self.handle, key.encode(), ctypes.byref(vt), ctypes.byref(et),
                                            ctypes.byref(n))):
            return None
        return vt.value, et.value, n.value

    def get_u32(self, key):
        v = ctypes.c_uint32()
        return None if _missing(lib().bb_gguf_get_u32(self.handle, key.encode(), ctypes.byref(v))) else v.value

    def get_f32(self, key):
        v = ctypes.c_float()
        return None if _missing(lib().bb_gguf_get_f32(self.handle, key.encode(), ctypes.byref(v))) else v.value

    def get_str(self, key):
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        if _missing(lib().bb_gguf_get_str(self.handle, key.encode(), ctypes.byref(p), ctypes.byref(n))):
            return None
        return ctypes.string_at(p.value, n.value).decode() if n.value else ""

    def get_u32_array(self, key):
        n = ctypes.c_size_t()
        if _missing(lib().bb_gguf_get_u32_array(self.handle, key.encode(), None, 0, ctypes.byref(n))):
            return None
        out = (ctypes.c_uint32 * max(n.value, 1))()
        check(lib().bb_gguf_get_u32_array(self.handle, key.encode(), out, n.value, ctypes.byref(n)))
        return [out[i] for i in range(n.value)]

    def get_str_array(self, key):
        t = self.meta_type(key)
        if t is None or t[0] != ARRAY:
            return None
        out, p, n = [], ctypes.c_void_p(), ctypes.c_size_t()
        for i in range(t[2]):
            if _missing(lib().bb_gguf_get_str_item(self.handle, key.encode(), i, ctypes.byref(p), ctypes.byref(n))):
                return None
            out.append(ctypes.string_at(p.value, n.value).decode() if n.value else "")
        return out

    def architecture(self):
        return self.get_str("general.architecture")

    def validate(self):
        """config::validate (config.rs:51-89); raises BBError with the reference's message."""
        check(lib().bb_gguf_validate(self.handle))

    def check_tensors(self):
        """Model::check_tensors (model.rs:572-584); returns the expected list's length."""
        n = ctypes.c_size_t()
        check(lib().bb_gguf_check_tensors(self.handle, ctypes.byref(n)))
        return n.value


# ---- writer ----------------------------------------------------------------------------------------

def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vt, v):
    if vt == STRING:
        return _str(v)
    if vt == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, it) for it in items)
    return struct.pack(_SCALAR[vt], v)


class GgufWriter:
    """Writes a GGUF (version 3): metadata key/values, then the tensor table, then the data
    section at the next `alignment` boundary with every tensor's data aligned as well."""

    def __init__(self, alignment=32, version=3):
        self.alignment, self.version = alignment, version
        self.meta, self.tensors = [], []

    def add(self, key, vt, value):
        """value: a Python scalar / str, or (elem_type, items) for ARRAY."""
        self.meta.append((key, vt, value))

    def add_tensor(self, name, dims, ggml_type, data):
        """dims in GGUF order (fastest-varying first); data: anything exposing the buffer protocol."""
        self.tensors.append((name, list(dims), ggml_type, memoryview(np.ascontiguousarray(data)).cast("B")))

    def _layout(self):
        head = [b"GGUF", struct.pack("<IQQ", self.version, len(self.tensors), len(self.meta))]
        head += [_str(k) + struct.pack("<I", vt) + _value(vt, v) for k, vt, v in self.meta]
        offsets, off = [], 0
        for name, dims, ty, data in self.tensors:
            offsets.append(off)
            off = -(-(off + data.nbytes) // self.alignment) * self.alignment
        for (name, dims, ty, data), o in zip(self.tensors, offsets):
            head.append(_str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
                        + struct.pack("<IQ", ty, o))
        head = b"".join(head)
        head += b"\0" * (-len(head) % self.alignment)
        return head, offsets

    def write(self, f):
        head, offsets = self._layout()
        f.write(head)
        pos = 0
        for (name, dims, ty, data), o in zip(self.tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(data)
            pos = o + data.nbytes

    def to_bytes(self):
        import io
        b = io.BytesIO()
        self.write(b)
        return b.getvalue()

    def save(self, path):
        with open(path, "wb") as f:
            self.write(f)


__all__ = ["GgufFile", "GgufWriter", "TensorInfo", "BBError"]
