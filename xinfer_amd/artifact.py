"""`.xinfer` artifacts: writer, reader and device loading of INT4 projections.

Python mirror of the reference's artifact layer over the C-ABI of
include/xinfer_hip/xinfer_artifact.h:

* ``ArtifactWriter``  -- src/artifact/writer.h:11-40, writer.cpp:20-191
  (same layout: 64-byte header, metadata, 64-byte-aligned sections, section
  table, 16-byte footer with the CRC-64 of everything before it)
* ``ArtifactReader``  -- src/artifact/reader.h:12-61 (open / close / header /
  footer / raw_metadata_json / list_sections / has_section /
  get_section_info / read_section / validate_checksum) plus
  ``upload_section`` (device copy verified by a GPU CRC-64)
* ``load_linear``     -- src/targets/qwen3_8_27b/weights.cpp:252-303
* ``crc64`` / ``crc64_file`` -- src/artifact/c_api.h:14-18

Errors raise ``ArtifactError`` carrying the status and the reader's message
(the reference returns false with an error string).
"""
from __future__ import annotations

import ctypes
import enum
import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

from . import _lib

MAGIC_BYTES = b"XINFER\0\0"            # container.h:11
FOOTER_MAGIC_BYTES = b"XINFFOOT"        # container.h:14
CURRENT_FORMAT_VERSION = 1              # container.h:16
SECTION_ALIGNMENT = 64                  # container.h:17
MAX_SECTION_NAME_LEN = 96               # container.h:18


class SectionType(enum.IntEnum):
    """container.h:19-27."""
    RawBlob = 0x0000
    MetadataJson = 0x0001
    TokenizerData = 0x0002
    TensorWeights = 0x0003
    TensorScales = 0x0004
    ChatTemplate = 0x0005
    Custom = 0x00FF


class ArtifactError(RuntimeError):
    def __init__(self, what: str, status: int, message: str = ""):
        self.status = status
        self.message = message
        super().__init__(f"{what}: {message or status}")


@dataclass
class SectionInfo:
    """A section table entry (container.h:50-58)."""
    name: str
    type_tag: int
    flags: int
    offset: int
    size: int
    checksum: int


@dataclass
class LinearWeightView:
    """weights.h:13-23: device tensors of one INT4 projection."""
    weights_int4: object  # torch uint8 [out_features, in_features // 2] on the device
    scales: object        # torch float16 [out_features, in_features // group_size]
    in_features: int
    out_features: int
    group_size: int = 128

    def is_valid(self) -> bool:
        return self.weights_int4 is not None and self.scales is not None


def _L():
    return _lib.load_library()


def crc64(data) -> int:
    """CRC-64/ECMA-182 (reflected) of a bytes-like object (c_api.h:15)."""
    mv = memoryview(data).cast("B")
    if mv.nbytes == 0:
        return 0
    buf = (ctypes.c_uint8 * mv.nbytes).from_buffer_copy(mv) if mv.readonly else \
        (ctypes.c_uint8 * mv.nbytes).from_buffer(mv)
    return int(_L().xinfer_crc64(ctypes.addressof(buf), mv.nbytes))


def crc64_file(path: str, max_bytes: int = 0) -> int:
    """CRC-64 of a file's first max_bytes bytes (0: all) (c_api.h:18)."""
    return int(_L().xinfer_crc64_file(os.fsencode(path), max_bytes))


def crc64_device(t, nbytes: Optional[int] = None, stream=None) -> int:
    """CRC-64 of a device tensor's bytes, computed on the GPU (blocks on the result)."""
    import torch
    n = t.numel() * t.element_size() if nbytes is None else nbytes
    out = torch.zeros(1, dtype=torch.int64, device=t.device)
    s = stream if stream is not None else torch.cuda.current_stream(t.device).cuda_stream
    _lib.check("xinfer_crc64_device",
               _L().xinfer_crc64_device(ctypes.c_void_p(s), ctypes.c_void_p(t.data_ptr()), n,
                                        ctypes.c_void_p(out.data_ptr()), None, 0))
    return int(out.cpu().item()) & 0xFFFFFFFFFFFFFFFF


# ----------------------------------------------------------------- writer ----

class ArtifactWriter:
    """writer.h:11-40.  Sections keep insertion order; names are unique,
    non-empty and shorter than 96 bytes (writer.cpp:20-31)."""

    def __init__(self):
        self._meta = b""
        self._sections: List[Tuple[str, int, int, bytes]] = []

    def set_metadata(self, metadata: Dict) -> None:
        """Metadata as a JSON object (model_name, quant_scheme, tokenizer_type,
        properties: the fields of ArtifactMetadata, metadata.h:10-14)."""
        self._meta = json.dumps(metadata, separators=(",", ":")).encode()

    def set_raw_metadata_json(self, json_str) -> None:
        self._meta = json_str.encode() if isinstance(json_str, str) else bytes(json_str)

    def add_section(self, name: str, type_tag: int, data, flags: int = 0) -> bool:
        raw = name.encode()
        if not raw or len(raw) >= MAX_SECTION_NAME_LEN or any(s[0] == name for s in self._sections):
            return False
        self._sections.append((name, int(type_tag), int(flags), bytes(data)))
        return True

    def write_to_file(self, path: str) -> None:
        pad = lambda off: (SECTION_ALIGNMENT - off % SECTION_ALIGNMENT) % SECTION_ALIGNMENT  # noqa: E731
        entries = []
        with open(path, "wb") as f:
            f.write(b"\0" * 64)                      # header placeholder
            off = 64
            meta_off, meta_size = off, len(self._meta)
            f.write(self._meta)
            off += meta_size
            for name, tag, flags, data in self._sections:
                p = pad(off)
                f.write(b"\0" * p)
                off += p
                entries.append(struct.pack("<96sIIQQQ", name.encode(), tag, flags, off, len(data),
                                           crc64(data) if data else 0))
                f.write(data)
                off += len(data)
            p = pad(off)
            f.write(b"\0" * p)
            off += p
            table_off, table_size = off, 128 * len(entries)
            for e in entries:
                f.write(e)
            off += table_size
            header = struct.pack("<8sIIIIQQQQQ", MAGIC_BYTES, CURRENT_FORMAT_VERSION, 64, 0,
                                 len(entries), meta_off, meta_size, table_off, table_size, off + 16)
            f.seek(0)
            f.write(header)
        footer = struct.pack("<Q8s", crc64_file(path, off), FOOTER_MAGIC_BYTES)
        with open(path, "ab") as f:
            f.write(footer)


# ----------------------------------------------------------------- reader ----

_ERR = 1024


class ArtifactReader:
    """reader.h:12-61 over the C reader (xinfer_artifact_*)."""

    def __init__(self, path: Optional[str] = None):
        self._h = ctypes.c_void_p()
        if path is not None:
            self.open(path)

    def open(self, path: str) -> None:
        self.close()
        err = ctypes.create_string_buffer(_ERR)
        rc = _L().xinfer_artifact_open(os.fsencode(path), ctypes.byref(self._h), err, _ERR)
        if rc:
            self._h = ctypes.c_void_p()
            raise ArtifactError("open", rc, err.value.decode(errors="replace"))

    def close(self) -> None:
        if self._h:
            _L().xinfer_artifact_close(self._h)
            self._h = ctypes.c_void_p()

    def is_open(self) -> bool:
        return bool(self._h)

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _need(self):
        if not self._h:
            raise ArtifactError("reader", _lib.XINFER_ERR_INVALID_ARG, "ArtifactReader is not open.")

    def header(self) -> Dict:
        self._need()
        h = _lib.FileHeader()
        _lib.check("xinfer_artifact_header", _L().xinfer_artifact_header(self._h, ctypes.byref(h)))
        return {f: (bytes(getattr(h, f)) if f == "magic" else int(getattr(h, f))) for f, _ in h._fields_}

    def footer_checksum(self) -> int:
        self._need()
        v = ctypes.c_uint64()
        _lib.check("xinfer_artifact_footer", _L().xinfer_artifact_footer(self._h, ctypes.byref(v)))
        return int(v.value)

    def raw_metadata_json(self) -> str:
        self._need()
        n = ctypes.c_size_t()
        p = _L().xinfer_artifact_metadata_json(self._h, ctypes.byref(n))
        return ctypes.string_at(p, n.value).decode() if n.value else ""

    def metadata(self) -> Dict:
        raw = self.raw_metadata_json()
        try:
            return json.loads(raw) if raw else {}
        except ValueError:
            return {}

    def list_sections(self) -> List[str]:
        self._need()
        L = _L()
        out = []
        for i in range(L.xinfer_artifact_section_count(self._h)):
            e = _lib.SectionInfo()
            _lib.check("xinfer_artifact_section_at", L.xinfer_artifact_section_at(self._h, i, ctypes.byref(e)))
            out.append(e.name.decode())
        return out

    def get_section_info(self, name: str) -> Optional[SectionInfo]:
        self._need()
        e = _lib.SectionInfo()
        if _L().xinfer_artifact_section_by_name(self._h, name.encode(), ctypes.byref(e)):
            return None
        return SectionInfo(e.name.decode(), e.type_tag, e.flags, e.offset, e.size, e.checksum)

    def has_section(self, name: str) -> bool:
        return self.get_section_info(name) is not None

    def read_section(self, name: str) -> bytes:
        """Payload on the host, CRC-64 checked (reader.cpp:225-276)."""
        info = self.get_section_info(name)
        size = info.size if info else 0
        buf = ctypes.create_string_buffer(max(1, size))
        err = ctypes.create_string_buffer(_ERR)
        rc = _L().xinfer_artifact_read_section(self._h, name.encode(), buf, size, err, _ERR)
        if rc:
            raise ArtifactError("read_section", rc, err.value.decode(errors="replace"))
        return buf.raw[:size]

    def validate_checksum(self) -> None:
        """Whole-file CRC-64 against the footer (reader.cpp:278-318)."""
        self._need()
        err = ctypes.create_string_buffer(_ERR)
        rc = _L().xinfer_artifact_validate_checksum(self._h, err, _ERR)
        if rc:
            raise ArtifactError("validate_checksum", rc, err.value.decode(errors="replace"))

    def upload_section(self, name: str, dst, verify: bool = True, stream=None) -> None:
        """Copy a section into device tensor `dst` (>= section size bytes) and,
        with verify, check its CRC-64 on the GPU."""
        import torch
        self._need()
        s = stream if stream is not None else torch.cuda.current_stream(dst.device).cuda_stream
        err = ctypes.create_string_buffer(_ERR)
        rc = _L().xinfer_artifact_upload_section(self._h, name.encode(), ctypes.c_void_p(s),
                                                 ctypes.c_void_p(dst.data_ptr()),
                                                 dst.numel() * dst.element_size(), int(verify), err, _ERR)
        if rc:
            raise ArtifactError("upload_section", rc, err.value.decode(errors="replace"))


def load_linear(reader: ArtifactReader, weight_name: str, out_features: int, in_features: int,
                group_size: int = 128, device="cuda") -> LinearWeightView:
    """weights.cpp:252-303: `weight_name` and `weight_name + ".scales"` into
    device tensors, sizes checked as there, CRC-64 verified on the GPU."""
    import torch
    w_bytes = out_features * (in_features // 2)
    s_bytes = out_features * (in_features // group_size) * 2
    for name, want, what in ((weight_name, w_bytes, "Weight"), (weight_name + ".scales", s_bytes, "Scales")):
        info = reader.get_section_info(name)
        if info is None:
            raise ArtifactError("load_linear", _lib.XINFER_ERR_INVALID_ARG, f"Section not found: {name}")
        if info.size != want:
            raise ArtifactError("load_linear", _lib.XINFER_ERR_IO,
                                f"{what} size mismatch for {name}: expected {want}, got {info.size}")
    W = torch.empty((out_features, in_features // 2), dtype=torch.uint8, device=device)
    S = torch.empty((out_features, in_features // group_size), dtype=torch.float16, device=device)
    reader.upload_section(weight_name, W)
    reader.upload_section(weight_name + ".scales", S)
    return LinearWeightView(W, S, in_features, out_features, group_size)
