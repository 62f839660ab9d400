"""The .cmf v2 model container (crates/cortiq-core/src/format.rs) over the
native reader of libcmfhip (csrc/container.cpp, include/cmf_hip.h).

`CmfFile.open(path)` mirrors `CmfModel::open` (format.rs:390-584): the file is
mapped read-only and validated strictly (envelope, header JSON, tensor
directory, per-tensor bounds and lengths, unique names); any inconsistency
raises the matching `CmfFileError` subclass, as the reference returns a
`CmfError` variant.  Tensor bytes are zero-copy views of the mapping.
`open_sharded` (format.rs:589-650), `verify` (:1063-1110) and `tensor_index`
(:809-821) keep the reference's names and behaviour.

The masks, vocab and sparse-index sections are exposed as raw bytes only
(their decoders serve task masks and the tokenizer, outside the decode path).
"""
import ctypes as C
import json
import os

import numpy as np

from . import CmfError, FileSections, FileTensor, lib


class CmfFileError(CmfError):
    """A .cmf file failed validation (format.rs CmfError)."""


class FileNotFound(CmfFileError):
    pass


class InvalidMagic(CmfFileError):
    pass


class UnsupportedVersion(CmfFileError):
    pass


class UnsupportedFeature(CmfFileError):
    pass


class BoundsError(CmfFileError):
    pass


class ParseError(CmfFileError):
    pass


class UnknownDtype(CmfFileError):
    pass


class IoError(CmfFileError):
    pass


class MissingTensor(CmfFileError):
    pass


_KINDS = {-2: FileNotFound, -3: InvalidMagic, -4: UnsupportedVersion, -5: UnsupportedFeature,
          -6: BoundsError, -7: ParseError, -8: UnknownDtype, -9: IoError, -10: MissingTensor}

# TensorDtype ids and names (cortiq-core/src/types.rs:10-160)
DTYPE_NAMES = {0: "f32", 1: "f16", 2: "bf16", 3: "q8_row", 4: "q4_block", 5: "mix84", 6: "u8", 7: "q4_col",
               8: "vbit", 9: "q8_2f", 10: "vbit_ro", 11: "q4_tiled", 12: "q1", 13: "q1s", 14: "q1t",
               15: "q4_tiled_p", 16: "q2_tiled_p"}
SECTIONS = ("header", "dir", "data", "masks", "vocab", "index")


def _check(rc):
    if rc < 0:
        raise _KINDS.get(rc, CmfError)(lib().cmf_last_error().decode())
    return rc


def hash64(data):
    """hash64 (cortiq-core/src/hash.rs) of a bytes-like object."""
    b = np.frombuffer(memoryview(data).cast("B"), dtype=np.uint8) if not isinstance(data, np.ndarray) else \
        np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    return int(lib().cmf_hash64(b.ctypes.data_as(C.c_void_p) if b.size else None, b.size))


class TensorEntry:
    """One directory record (TensorEntry, format.rs:255-269)."""
    __slots__ = ("name", "dtype", "shape", "off", "nbytes", "hash", "shard", "index")

    def __init__(self, name, dtype, shape, off, nbytes, hash_, shard, index):
        self.name, self.dtype, self.shape = name, dtype, shape
        self.off, self.nbytes, self.hash, self.shard, self.index = off, nbytes, hash_, shard, index

    @property
    def n_elems(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def dtype_name(self):
        return DTYPE_NAMES[self.dtype]

    def __repr__(self):
        return f"TensorEntry({self.name!r}, {self.dtype_name}, {list(self.shape)}, off={self.off}, nbytes={self.nbytes})"


def _view(addr, n, owner):
    """uint8 array over n bytes of the mapping at addr; keeps owner alive."""
    if n == 0:
        return np.zeros(0, dtype=np.uint8)
    buf = (C.c_uint8 * n).from_address(addr)
    buf._owner = owner  # the mapping lives as long as any view of it
    a = np.frombuffer(buf, dtype=np.uint8)
    a.flags.writeable = False
    return a


class CmfFile:
    """An open .cmf v2 file: header (dict), tensor directory, zero-copy
    tensor bytes."""

    def __init__(self, path, _handle=None):
        self.path = os.fspath(path)
        h = C.c_void_p()
        if _handle is None:
            _check(lib().cmf_file_open(self.path.encode(), C.byref(h)))
        else:
            h = _handle
        self._h = h
        try:
            self._load_meta()
        except Exception:
            self.close()
            raise

    @classmethod
    def open(cls, path):
        return cls(path)

    def _load_meta(self):
        s = FileSections()
        _check(lib().cmf_file_info(self._h, C.byref(s)))
        self.required_features = int(s.required_features)
        self.sections = {n: (int(s.off[i]), int(s.len[i])) for i, n in enumerate(SECTIONS)}
        self._base, self.file_len = int(s.base), int(s.file_len)
        off, ln = self.sections["header"]
        try:
            self.header = json.loads(bytes(_view(self._base + off, ln, self)).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise ParseError(f"header JSON: {e}") from None
        # CmfHeader's fields without a serde default (format.rs:78-125)
        for k in ("version", "arch", "quant_type"):
            if k not in self.header:
                raise ParseError(f"header JSON: missing field `{k}`")
        if not isinstance(self.header["arch"], dict):
            raise ParseError("header JSON: `arch` is not an object")
        self._read_dir()

    def _read_dir(self):
        n = _check(lib().cmf_file_count(self._h))
        ents = []
        e = FileTensor()
        for i in range(n):
            _check(lib().cmf_file_entry(self._h, i, C.byref(e)))
            name = C.string_at(e.name, e.name_len).decode("utf-8")
            ents.append(TensorEntry(name, e.dtype, tuple(int(e.shape[k]) for k in range(e.ndim)), int(e.off),
                                    int(e.nbytes), int(e.hash), int(e.shard), i))
        self.tensors = ents

    @property
    def arch(self):
        return self.header["arch"]

    def tensor_index(self, name):
        b = name.encode("utf-8")
        rc = lib().cmf_file_find(self._h, b, len(b))
        return None if rc < 0 else rc

    def tensor(self, name):
        i = self.tensor_index(name)
        return None if i is None else self.tensors[i]

    def entry_bytes(self, entry):
        """The tensor's payload (entry_bytes, format.rs:924-933): a read-only
        view of the file mapping."""
        e = FileTensor()
        _check(lib().cmf_file_entry(self._h, entry.index, C.byref(e)))
        return _view(int(e.data or 0), int(e.nbytes), self)

    def tensor_bytes(self, name):
        i = self.tensor_index(name)
        if i is None:
            raise MissingTensor(f"tensor '{name}' not found in CMF directory")
        return self.entry_bytes(self.tensors[i])

    def section_bytes(self, name):
        off, ln = self.sections[name]
        return _view(self._base + off, ln, self)

    @property
    def vocab(self):
        """The embedded tokenizer.json bytes, or None (format.rs:545-550)."""
        return bytes(self.section_bytes("vocab")) if self.sections["vocab"][1] else None

    def dir_hash(self):
        """hash64 of the tensor directory stored in the envelope (format.rs:856-858)."""
        return int(self._info().dir_hash)

    def _info(self):
        s = FileSections()
        _check(lib().cmf_file_info(self._h, C.byref(s)))
        return s

    def verify(self):
        """Integrity problems (verify, format.rs:1063-1110): envelope header /
        directory hashes, the optional sections' hashes from the header's
        section_hashes, every tensor's hash.  Empty = intact."""
        sh = self.header.get("section_hashes") or {}
        stored = (C.c_uint64 * 3)()
        malformed = {}
        for i, name in enumerate(("masks", "vocab", "index")):
            hx = sh.get(name)
            if hx is None:
                continue
            v = _parse_u64_hex(hx)
            if v is None:
                malformed[name] = f"section '{name}': malformed hash '{hx}'"
            else:
                stored[i] = v
        cap = 1 << 20
        buf = C.create_string_buffer(cap)
        n = C.c_int()
        _check(lib().cmf_file_verify(self._h, stored, buf, cap, C.byref(n)))
        lines = buf.value.decode().split("\n") if n.value else []
        out = [l for l in lines if l.startswith(("section 'header'", "section 'dir'"))]
        for name in ("masks", "vocab", "index"):
            if name in malformed:
                out.append(malformed[name])
            out += [l for l in lines if l.startswith(f"section '{name}'")]
        out += [l for l in lines if l.startswith("tensor ")]
        return out

    @classmethod
    def open_sharded(cls, path):
        """Open shard 1 of a sharded model and merge its siblings'
        directories (open_sharded, format.rs:589-650); a file without shard
        coordinates opens as usual."""
        first = cls(path)
        info = first.header.get("shard")
        if info is None:
            return first
        try:
            no, count = int(info["no"]), int(info["count"])
            if no != 1:
                raise ParseError(f"open shard 1, not {no} (of {count})")
            name = os.path.basename(first.path)
            tag1 = f"-{1:05d}-of-{count:05d}.cmf"
            if not name.endswith(tag1):
                raise ParseError(f"shard file must end with '{tag1}' (got '{name}')")
            stem = os.path.join(os.path.dirname(first.path), name[: len(name) - len(tag1)])
            for k in range(2, count + 1):
                sib = f"{stem}-{k:05d}-of-{count:05d}.cmf"
                sh = cls(sib)
                si = sh.header.get("shard")
                if not (isinstance(si, dict) and si.get("no") == k and si.get("count") == count):
                    sh.close()
                    raise ParseError(f"{sib}: wrong shard coords {si!r}")
                rc = lib().cmf_file_attach_shard(first._h, sh._h)
                if rc < 0:
                    sh.close()
                    _check(rc)
                sh._h = None  # consumed by the attach
            first._read_dir()
            return first
        except Exception:
            first.close()
            raise

    def close(self):
        if getattr(self, "_h", None):
            lib().cmf_file_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


def _parse_u64_hex(s):
    """u64::from_str_radix(s, 16): an optional '+', then hex digits only."""
    if not isinstance(s, str):
        return None
    d = s[1:] if s.startswith("+") else s
    if not d or any(c not in "0123456789abcdefABCDEF" for c in d):
        return None
    v = int(d, 16)
    return v if v < 1 << 64 else None


def _f16_to_f32(u16):
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float32)


def dequant_vector(entry, raw):
    """f32 values of an f32 / f16 / bf16 tensor (dequant_tensor's float arms,
    quant.rs): f16 converts exactly, bf16 is the upper half of an f32."""
    n = entry.n_elems
    if entry.dtype == 0:
        return np.frombuffer(raw, dtype="<f4", count=n).astype(np.float32)
    if entry.dtype == 1:
        return _f16_to_f32(np.frombuffer(raw, dtype="<u2", count=n))
    if entry.dtype == 2:
        return (np.frombuffer(raw, dtype="<u2", count=n).astype(np.uint32) << 16).view(np.float32)
    raise CmfError(f"tensor '{entry.name}': dtype {entry.dtype_name} is not a float vector")
