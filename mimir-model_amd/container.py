"""Opening a mim container and uploading its weights to the GPU.

The reader follows the reference's `file.go` as specified in
spec/container.md (v0.2): it validates the preamble, the index (header,
section table, tensor table, string pool) and the canonical packing of the
weights section in the spec's order, and reports the first fault with the
spec's error code (`MimError.code`, section 9). The metadata section is
decoded as spec/metadata.md defines it. Nothing of the file is parsed past
the index until it has been validated; tensor bytes are read in place from a
read-only mapping.

`MimFile.upload()` copies the whole weights section to the device in one
transfer (the reference's `File.Weights()`, file.go:401-404, and the
loading guidance of container.md section 7) and registers every quantized
matrix as a view at its offset, so no tensor is copied twice.

Host-side code: it decides nothing about results. The decoder and its
kernels live in libmimg.
"""
import hashlib
import mmap
import struct

import numpy as np

PREAMBLE = 64
INDEX_HEADER = 16
SECTION_ENTRY = 64
TENSOR_ENTRY = 96
MAX_INDEX = 256 << 20
MAX_POOL = 256 << 20
MIN_ALIGN, MAX_ALIGN = 4096, 16 << 20
SECTION_ALIGN = 8
MAX_RANK = 8
MAX_NAME = 4096
TENSOR_ALIGN, LARGE_TENSOR_ALIGN, LARGE_TENSOR = 64, 4096, 1 << 20
FLAG_REQUIRED = 1
KIND_WEIGHTS, KIND_METADATA, KIND_GRAPH, KIND_REPACK, KIND_TRAINING = 1, 2, 3, 4, 5

# spec/dtypes.md: id -> (name, block elements, block bytes)
DTYPES = {
    1: ("f32", 1, 4), 2: ("f16", 1, 2), 3: ("bf16", 1, 2), 4: ("f64", 1, 8), 5: ("i8", 1, 1), 6: ("u8", 1, 1),
    7: ("i16", 1, 2), 8: ("u16", 1, 2), 9: ("i32", 1, 4), 10: ("u32", 1, 4), 11: ("i64", 1, 8), 12: ("u64", 1, 8),
    13: ("bool", 1, 1), 14: ("f8_e4m3", 1, 1), 15: ("f8_e5m2", 1, 1),
    64: ("q8_0", 32, 34), 65: ("q4_0", 32, 18), 66: ("q4_k", 256, 144), 67: ("q6_k", 256, 210),
    68: ("mxfp4", 32, 17), 69: ("affine4_g64", 64, 36),
}
U64_MAX = (1 << 64) - 1


class MimError(ValueError):
    def __init__(self, code, msg):
        super().__init__(f"{code}: {msg}")
        self.code = code


def _in_bounds(off, ln, size):
    return off <= size and ln <= size - off


class Tensor:
    def __init__(self, name, dtype, shape, offset, length):
        self.name, self.dtype, self.shape, self.offset, self.length = name, dtype, shape, offset, length


class MimFile:
    """A validated mim container, mapped read-only."""

    def __init__(self, path):
        self._f = open(path, "rb")
        size = self._f.seek(0, 2)
        self.size = size
        self._m = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ) if size else b""
        self.buf = memoryview(self._m) if size else memoryview(b"")
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    def close(self):
        try:
            self.buf.release()
            if isinstance(self._m, mmap.mmap):
                self._m.close()
        except BufferError:
            pass  # arrays still view the mapping; it closes when they go
        self._f.close()

    # ---- parsing, in the order of spec/container.md section 9 -------------

    def _parse(self):
        b, size = self.buf, self.size
        if size < PREAMBLE:
            raise MimError("truncated", f"file of {size} bytes")
        magic = bytes(b[0:4])
        if magic not in (b"MIM\0", b"MMF\0"):
            raise MimError("bad-magic", repr(magic))
        major, minor, bom, align = struct.unpack_from("<HHII", b, 4)
        if bom == 0x0D0C0B0A:
            raise MimError("big-endian", "byte order mark")
        if bom != 0x0A0B0C0D:
            raise MimError("bad-byte-order-mark", hex(bom))
        if major != 0:
            raise MimError("unsupported-version", f"major {major}")
        ioff, ilen, doff, dlen, flen, reserved = struct.unpack_from("<6Q", b, 16)
        if align & (align - 1) or not MIN_ALIGN <= align <= MAX_ALIGN:
            raise MimError("bad-alignment", f"{align}")
        if flen > size:
            raise MimError("truncated", f"file length {flen} > {size}")
        if flen < size:
            raise MimError("bad-length", f"file length {flen} < {size}")
        if ioff < PREAMBLE or ioff % SECTION_ALIGN:
            raise MimError("misaligned", f"index offset {ioff}")
        if ilen > MAX_INDEX:
            raise MimError("index-too-large", f"{ilen}")
        if not _in_bounds(ioff, ilen, size):
            raise MimError("out-of-bounds", "index")
        if doff % align:
            raise MimError("misaligned", f"data offset {doff}")
        if not _in_bounds(doff, dlen, size):
            raise MimError("out-of-bounds", "weights")
        if reserved != 0:
            raise MimError("reserved-non-zero", "preamble bytes 56..63")
        self.major, self.minor, self.data_alignment = major, minor, align
        self.data_offset, self.data_length = doff, dlen

        if ilen < INDEX_HEADER:
            raise MimError("truncated", "index header")
        ns, nt, pool = struct.unpack_from("<IIQ", b, ioff)
        if pool > MAX_POOL or ilen != INDEX_HEADER + SECTION_ENTRY * ns + TENSOR_ENTRY * nt + pool:
            raise MimError("bad-length", "index length")
        pool_off = ioff + INDEX_HEADER + SECTION_ENTRY * ns + TENSOR_ENTRY * nt

        self.sections = {}
        regions = [(0, PREAMBLE), (ioff, ilen)]
        seen = set()
        p = ioff + INDEX_HEADER
        for _ in range(ns):
            kind, flags, off, ln, halg = struct.unpack_from("<IIQQB", b, p)
            rsv = bytes(b[p + 25:p + 32])
            digest = bytes(b[p + 32:p + 64])
            p += SECTION_ENTRY
            if flags & ~FLAG_REQUIRED:
                raise MimError("reserved-non-zero", "section flags")
            if any(rsv):
                raise MimError("reserved-non-zero", "section entry bytes 25..31")
            if halg not in (0, 1):
                raise MimError("bad-hash-algorithm", f"{halg}")
            if halg == 0 and any(digest):
                raise MimError("reserved-non-zero", "hash bytes with algorithm 0")
            known = 1 <= kind <= 5
            if known:
                if kind in seen:
                    raise MimError("duplicate", f"section kind {kind}")
                seen.add(kind)
            elif flags & FLAG_REQUIRED:
                raise MimError("unknown-required-section", f"kind {kind}")
            if not _in_bounds(off, ln, size):
                raise MimError("out-of-bounds", f"section kind {kind}")
            if kind == KIND_WEIGHTS:
                if off != doff or ln != dlen:
                    raise MimError("bad-length", "weights section entry and preamble disagree")
            elif off % SECTION_ALIGN:
                raise MimError("misaligned", f"section kind {kind} at {off}")
            regions.append((off, ln))
            if known:
                self.sections[kind] = (off, ln, halg, digest)
        if KIND_WEIGHTS not in self.sections:
            raise MimError("missing-section", "weights")
        regions.sort()
        end = 0
        for off, ln in regions:
            if off < end:
                raise MimError("overlap", f"region at {off}")
            end = max(end, off + ln)

        self.tensors = []
        prev = None
        for _ in range(nt):
            no, nl, dt, rank = struct.unpack_from("<IIIB", b, p)
            rsv = bytes(b[p + 13:p + 16])
            dims = struct.unpack_from("<8Q", b, p + 16)
            toff, tlen = struct.unpack_from("<QQ", b, p + 80)
            p += TENSOR_ENTRY
            if not _in_bounds(no, nl, pool):
                raise MimError("out-of-bounds", "tensor name")
            raw = bytes(b[pool_off + no:pool_off + no + nl])
            try:
                name = raw.decode("utf-8")
            except UnicodeDecodeError:
                raise MimError("bad-name", repr(raw)) from None
            if not 1 <= nl <= MAX_NAME:
                raise MimError("bad-name", f"length {nl}")
            if prev is not None:
                if raw == prev:
                    raise MimError("duplicate", name)
                if raw < prev:
                    raise MimError("unsorted", name)
            prev = raw
            if dt not in DTYPES:
                raise MimError("bad-dtype", f"{dt} ({name})")
            if any(rsv):
                raise MimError("reserved-non-zero", "tensor entry bytes 13..15")
            if rank > MAX_RANK:
                raise MimError("bad-shape", f"rank {rank} ({name})")
            if any(dims[rank:]):
                raise MimError("reserved-non-zero", "unused dims")
            shape = list(dims[:rank])
            _, be, bb = DTYPES[dt]
            if be > 1 and (rank == 0 or shape[-1] % be):
                raise MimError("bad-shape", f"{shape} for blocks of {be} ({name})")
            elems = 1
            for d in shape:
                elems *= d
                if elems > U64_MAX:
                    raise MimError("overflow", f"elements of {name}")
            want = elems // be * bb
            if want > U64_MAX:
                raise MimError("overflow", f"bytes of {name}")
            if tlen != want:
                raise MimError("size-mismatch", f"{name}: {tlen} bytes, {want} expected")
            a = LARGE_TENSOR_ALIGN if tlen >= LARGE_TENSOR else TENSOR_ALIGN
            if toff % a:
                raise MimError("misaligned", f"{name} at {toff}")
            if not _in_bounds(toff, tlen, dlen):
                raise MimError("out-of-bounds", f"{name} data")
            self.tensors.append(Tensor(name, dt, shape, toff, tlen))

        # canonical packing (section 6.4)
        end = 0
        for t in sorted(self.tensors, key=lambda t: (t.offset, t.length)):
            if t.offset < end:
                raise MimError("overlap", t.name)
            a = LARGE_TENSOR_ALIGN if t.length >= LARGE_TENSOR else TENSOR_ALIGN
            if t.offset != (end + a - 1) // a * a:
                raise MimError("non-canonical-layout", t.name)
            end = t.offset + t.length
        if end != dlen:
            raise MimError("non-canonical-layout", "the weights section does not end at the last tensor")
        self.by_name = {t.name: t for t in self.tensors}

    # ---- access ------------------------------------------------------------

    def weights(self):
        """The weights section, in place (File.Weights)."""
        return self.buf[self.data_offset:self.data_offset + self.data_length]

    def tensor_bytes(self, name):
        t = self.by_name[name]
        return self.buf[self.data_offset + t.offset:self.data_offset + t.offset + t.length]

    def verify_hashes(self):
        """SHA-256 of every section that carries one (VerifyHashes)."""
        for kind, (off, ln, halg, digest) in self.sections.items():
            if halg == 1 and hashlib.sha256(self.buf[off:off + ln]).digest() != digest:
                raise MimError("hash-mismatch", f"section kind {kind}")

    def metadata(self):
        """The metadata section (spec/metadata.md) as {key: value}."""
        if KIND_METADATA not in self.sections:
            return {}
        off, ln, _, _ = self.sections[KIND_METADATA]
        b = self.buf[off:off + ln]
        if ln < 16 or bytes(b[0:4]) not in (b"MIMM", b"MMFM"):
            raise MimError("bad-metadata", "magic")
        count, pool = struct.unpack_from("<IQ", b, 4)
        if count > 1 << 24 or ln != 16 + 32 * count + pool:
            raise MimError("bad-metadata", "length")
        pb = 16 + 32 * count

        def pool_bytes(o, n):
            if not _in_bounds(o, n, pool):
                raise MimError("bad-metadata", "pool bounds")
            return bytes(b[pb + o:pb + o + n])

        out = {}
        for i in range(count):
            ko, kl, typ, cnt, payload = struct.unpack_from("<IIB3xIQ", b, 16 + 32 * i)
            key = pool_bytes(ko, kl).decode("utf-8")
            if typ == 1:
                v = struct.unpack("<q", struct.pack("<Q", payload))[0]
            elif typ == 2:
                v = payload
            elif typ == 3:
                v = struct.unpack("<d", struct.pack("<Q", payload))[0]
            elif typ == 4:
                v = bool(payload)
            elif typ == 5:
                v = pool_bytes(payload, cnt).decode("utf-8")
            elif typ == 6:
                v = pool_bytes(payload, cnt)
            elif typ == 7:
                v = list(struct.unpack(f"<{cnt}q", pool_bytes(payload, 8 * cnt)))
            elif typ == 8:
                v = list(struct.unpack(f"<{cnt}d", pool_bytes(payload, 8 * cnt)))
            elif typ == 9:
                tab = struct.unpack(f"<{2 * cnt}I", pool_bytes(payload, 8 * cnt))
                v = [pool_bytes(tab[2 * j], tab[2 * j + 1]).decode("utf-8") for j in range(cnt)]
            else:
                raise MimError("bad-metadata", f"type {typ} of {key}")
            out[key] = v
        return out

    def llama_config(self, context=0):
        """The decoder shape from the metadata an import writes (reference
        importer/llama.go LlamaConfigOf); the cache length is the file's
        `mim.context_length` unless given."""
        import decoder

        md = self.metadata()
        return decoder.config_from_metadata(md, context or md.get("mim.context_length", 0))

    def upload(self):
        """The weights section to the device in one transfer, and every
        tensor as decoder input: quantized matrices as views into the
        uploaded section, f32 vectors read in place."""
        import mimg

        sec = mimg.WeightsSection(np.frombuffer(self.weights(), np.uint8))
        tensors = {}
        for t in self.tensors:
            if t.dtype in (64, 66, 67) and len(t.shape) == 2:
                tensors[t.name] = (t.dtype, t.shape, sec.view(t.offset, t.length, t.dtype, t.shape[0], t.shape[1]))
            elif t.dtype == 1 and len(t.shape) == 1:
                tensors[t.name] = (1, t.shape, np.frombuffer(self.tensor_bytes(t.name), np.float32).copy())
        return sec, tensors
