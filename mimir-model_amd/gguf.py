"""Reading a GGUF model for the GPU decoder, as the reference's importer
reads one (importer/gguf.go ParseGGUF, importer/llama.go LlamaConfigOf).

GGUF v2 and v3, little-endian: the header, the metadata (scalars and arrays
decoded to the same Python types the reference's metadata holds, with its
limits on counts, string sizes, nesting and decoded size), the tensor
table (ggml types mapped to mim dtypes, dimensions reversed to mim's
outermost-first order, byte sizes from the dtype, offsets aligned to
`general.alignment`), and the data region. Errors carry the reference's
messages' meaning (`GGUFError`).

`GGUFFile.upload()` copies the tensor data region to the device in one
transfer and registers each quantized matrix as a view at its offset; the
norm scales and biases (f32) are read in place.
"""
import mmap
import struct

import numpy as np

import container

# ggml type -> mim dtype id (the block layouts are the same, spec/dtypes.md)
GGML_TYPES = {0: 1, 1: 2, 2: 65, 8: 64, 12: 66, 14: 67, 24: 5, 25: 7, 26: 9, 27: 11, 28: 4, 30: 3, 39: 68}
GGML_NAMES = {3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 9: "Q8_1", 10: "Q2_K", 11: "Q3_K", 13: "Q5_K", 15: "Q8_K",
              16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S",
              23: "IQ4_XS", 29: "IQ1_M", 34: "TQ1_0", 35: "TQ2_0"}
(U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64) = range(13)
MAX_COUNT = 1 << 24
MAX_STRING = 1 << 26
MAX_DEPTH = 8
MAX_METADATA = 64 << 20
MAX_KEY = 1024
MAX_RANK = 8
SCALAR = {U8: ("B", 1), I8: ("b", 1), U16: ("H", 2), I16: ("h", 2), U32: ("I", 4), I32: ("i", 4), F32: ("f", 4),
          BOOL: ("B", 1), U64: ("Q", 8), I64: ("q", 8), F64: ("d", 8)}


class GGUFError(ValueError):
    pass


class _Reader:
    def __init__(self, b):
        self.b, self.off, self.mem = b, 0, 0

    def take(self, n):
        if n > len(self.b) - self.off:
            raise GGUFError(f"gguf: truncated at offset {self.off} (need {n} bytes)")
        p = self.b[self.off:self.off + n]
        self.off += n
        return p

    def u(self, fmt, n):
        return struct.unpack("<" + fmt, self.take(n))[0]

    def str(self):
        n = self.u("Q", 8)
        if n > MAX_STRING:
            raise GGUFError(f"gguf: string of {n} bytes at offset {self.off}")
        raw = bytes(self.take(n))
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError:
            raise GGUFError(f"gguf: invalid UTF-8 string at offset {self.off}") from None

    def charge(self, n):
        if n > MAX_METADATA - self.mem:
            raise GGUFError(f"gguf: metadata needs more than {MAX_METADATA} bytes of memory")
        self.mem += n

    def scalar(self, t):
        if t == STRING:
            return self.str()
        if t not in SCALAR:
            raise GGUFError(f"gguf: unknown value type {t}")
        fmt, n = SCALAR[t]
        v = self.u(fmt, n)
        if t == BOOL:
            if v > 1:
                raise GGUFError(f"gguf: bool value {v}")
            return v == 1
        if t in (F32, F64):
            return float(v)
        return v

    def value(self, t, depth):
        """(value, ok): ok is False for values metadata cannot hold (nested
        arrays, u64 arrays beyond the int64 range): skipped, not errors."""
        if t != ARRAY:
            v = self.scalar(t)
            if isinstance(v, str):
                self.charge(len(v))
            return v, True
        if depth >= MAX_DEPTH:
            raise GGUFError(f"gguf: arrays nested more than {MAX_DEPTH} deep at offset {self.off}")
        et, n = self.u("I", 4), self.u("Q", 8)
        least = 8 if et in (STRING, ARRAY) else SCALAR.get(et, (None, 0))[1]
        if least == 0:
            raise GGUFError(f"gguf: unknown array element type {et}")
        if n > (len(self.b) - self.off) // least:
            raise GGUFError(f"gguf: array of {n} elements at offset {self.off} exceeds the file")
        if et == ARRAY:
            for _ in range(n):
                self.value(ARRAY, depth + 1)
            return None, False
        if et == STRING:
            self.charge(16 * n)
            out = []
            for _ in range(n):
                s = self.str()
                self.charge(len(s))
                out.append(s)
            return out, True
        if et in (F32, F64):
            self.charge(8 * n)
            return [self.scalar(et) for _ in range(n)], True
        if et == U8:
            self.charge(n)
            return bytes(self.take(n)), True
        self.charge(8 * n)
        vals = [self.scalar(et) for _ in range(n)]
        ok = all(not (isinstance(x, int) and x > (1 << 63) - 1) for x in vals)
        return [int(x) for x in vals], ok


class GTensor:
    def __init__(self, name, dtype, shape, offset, size):
        self.name, self.dtype, self.shape, self.offset, self.length = name, dtype, shape, offset, size


class GGUFFile:
    """A parsed GGUF file, mapped read-only (tensor data is not copied)."""

    def __init__(self, path):
        self._f = open(path, "rb")
        size = self._f.seek(0, 2)
        if size == 0:
            self._f.close()
            raise GGUFError("gguf: bad magic")
        self._m = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        self.buf = memoryview(self._m)
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    def close(self):
        try:
            self.buf.release()
            self._m.close()
        except BufferError:
            pass  # arrays still view the mapping; it closes when they go
        self._f.close()

    def _parse(self):
        b = self.buf
        r = _Reader(b)
        if bytes(r.take(4)) != b"GGUF":
            raise GGUFError("gguf: bad magic")
        version = r.u("I", 4)
        if version not in (2, 3):
            if version & 0xFFFF == 0:
                raise GGUFError("gguf: big-endian files are not supported")
            raise GGUFError(f"gguf: unsupported version {version}")
        nt, nkv = r.u("Q", 8), r.u("Q", 8)
        rest = len(b) - r.off
        if nt > MAX_COUNT or nkv > MAX_COUNT or nkv > rest // 13 or nt > rest // 24:
            raise GGUFError(f"gguf: {nt} tensors and {nkv} keys do not fit in the file")
        md, skipped, alignment = {}, [], 32
        for _ in range(nkv):
            key = r.str()
            t = r.u("I", 4)
            v, ok = r.value(t, 0)
            if key == "" or len(key.encode()) > MAX_KEY:
                raise GGUFError(f"gguf: invalid metadata key {key!r}")
            if key in md or key in skipped:
                raise GGUFError(f"gguf: duplicate metadata key {key!r}")
            if key == "general.alignment":
                if t not in (U8, U16, U32, U64) or v == 0 or v & (v - 1) or v > 1 << 20:
                    raise GGUFError(f"gguf: invalid general.alignment {v}")
                alignment = v
            if not ok:
                skipped.append(key)
                continue
            md[key] = v
        if skipped:
            md["import.skipped_keys"] = skipped
        md["import.gguf_version"] = version
        infos, names = [], set()
        for _ in range(nt):
            name = r.str()
            nd = r.u("I", 4)
            if nd > MAX_RANK:
                raise GGUFError(f"gguf: tensor {name!r} has {nd} dimensions")
            dims = [r.u("Q", 8) for _ in range(nd)]
            shape = dims[::-1]  # GGUF lists the innermost dimension first
            gt = r.u("I", 4)
            off = r.u("Q", 8)
            if name in names:
                raise GGUFError(f"gguf: duplicate tensor {name!r}")
            names.add(name)
            if gt not in GGML_TYPES:
                if gt in GGML_NAMES:
                    raise GGUFError(f"gguf: tensor {name!r} has type {GGML_NAMES[gt]}, which mim does not define")
                raise GGUFError(f"gguf: tensor {name!r} has unknown type {gt}")
            dt = GGML_TYPES[gt]
            _, be, bb = container.DTYPES[dt]
            if be > 1 and (nd == 0 or shape[-1] % be):
                raise GGUFError(f"gguf: tensor {name!r}: shape {shape} is not whole blocks of {be}")
            elems = 1
            for d in shape:
                elems *= d
            size = elems // be * bb
            if size > (1 << 63):
                raise GGUFError(f"gguf: tensor {name!r}: size overflows")
            if off % alignment:
                raise GGUFError(f"gguf: tensor {name!r} offset {off} is not aligned to {alignment}")
            infos.append(GTensor(name, dt, shape, off, size))
        start = (r.off + alignment - 1) // alignment * alignment
        if start > len(b):
            raise GGUFError("gguf: tensor data starts past the end of the file")
        data_len = len(b) - start
        for t in infos:
            if t.offset > data_len or t.length > data_len - t.offset:
                raise GGUFError(f"gguf: tensor {t.name!r} data [{t.offset}, +{t.length}) is outside the file")
        self.version, self.metadata, self.alignment = version, md, alignment
        self.data_start, self.data_length = start, data_len
        self.tensors = infos
        self.by_name = {t.name: t for t in infos}

    def tensor_bytes(self, name):
        t = self.by_name[name]
        return self.buf[self.data_start + t.offset:self.data_start + t.offset + t.length]

    def upload(self):
        """The tensor data region to the device in one transfer; quantized
        matrices as views at their offsets, f32 vectors read in place."""
        import mimg

        end = max((t.offset + t.length for t in self.tensors), default=0)
        sec = mimg.WeightsSection(np.frombuffer(self.buf[self.data_start:self.data_start + end], np.uint8))
        tensors = {}
        for t in self.tensors:
            if t.dtype in (64, 66, 67) and len(t.shape) == 2:
                tensors[t.name] = (t.dtype, t.shape, sec.view(t.offset, t.length, t.dtype, t.shape[0], t.shape[1]))
            elif t.dtype == 1 and len(t.shape) == 1:
                tensors[t.name] = (1, t.shape, np.frombuffer(self.tensor_bytes(t.name), np.float32).copy())
        return sec, tensors
