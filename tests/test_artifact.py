"""CPU tests of the .xinfer layer (include/xinfer_hip/xinfer_artifact.h):
CRC-64 against the oracle restatement of src/artifact/checksum.cpp and the
published CRC-64/XZ check value, the writer/reader round trip, the reader's
rejection of malformed and corrupted files (the checks of reader.cpp:56-318),
and, where oracle/_ref/artifact_ref was built from the reference sources,
files written by either side read by the other, byte for byte."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
from xinfer_amd import _lib, artifact
from xinfer_amd.artifact import ArtifactError, ArtifactReader, ArtifactWriter, SectionType

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    _lib.load_library()


def _rand(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


# ------------------------------------------------------------------- CRC ----

def test_crc64_check_value():
    # CRC-64/XZ (reflected ECMA-182, init and xorout all ones): check("123456789")
    assert oracle.crc64(b"123456789") == 0x995DC9BBDF1939FA
    assert artifact.crc64(b"123456789") == 0x995DC9BBDF1939FA
    assert artifact.crc64(b"") == 0          # c_api.cpp:10
    assert oracle.crc64(b"") == 0


def test_crc64_matches_oracle_all_sizes():
    # sizes around the 8-byte slicing step, plus multi-thread pieces (>= 16 MB)
    for n in list(range(0, 40)) + [255, 256, 4095, 65537, (8 << 20) + 3, (40 << 20) + 11]:
        d = _rand(n, n)
        assert artifact.crc64(d) == oracle.crc64(d), n


def test_crc64_file_and_prefix(tmp_path):
    d = _rand((20 << 20) + 7, 3)
    p = tmp_path / "blob.bin"
    p.write_bytes(d)
    assert artifact.crc64_file(str(p)) == oracle.crc64(d)
    for m in (1, 1000, (17 << 20) + 1):
        assert artifact.crc64_file(str(p), m) == oracle.crc64(d[:m])
    assert artifact.crc64_file(str(tmp_path / "missing.bin")) == 0  # c_api.cpp:17-18


# ------------------------------------------------------------ round trip ----

def _write(path, sections, meta='{"model_name":"m"}'):
    w = ArtifactWriter()
    w.set_raw_metadata_json(meta)
    for name, tag, data in sections:
        assert w.add_section(name, tag, data)
    w.write_to_file(str(path))


SECTIONS = [("model.embed_tokens.weight", SectionType.TensorWeights, _rand(128 * 1024 + 17, 1001)),
            ("model.layers.0.self_attn.q_proj.weight", SectionType.TensorWeights, _rand(256 * 1024 + 3, 1002)),
            ("model.layers.0.self_attn.q_proj.scales", SectionType.TensorScales, _rand(8 * 1024, 1003)),
            ("tokenizer.data", SectionType.TokenizerData, _rand(32 * 1024 + 42, 1004)),
            ("empty", SectionType.RawBlob, b"")]


def test_writer_reader_round_trip(tmp_path):
    p = tmp_path / "a.xinfer"
    meta = json.dumps({"model_name": "Qwen/Qwen3.8-27B", "quant_scheme": "INT4-G128-SYM",
                       "tokenizer_type": "qwen3_8_tiktoken", "properties": {"hidden_size": "5120"}})
    _write(p, SECTIONS, meta)
    with ArtifactReader(str(p)) as r:
        h = r.header()
        assert h["magic"] == b"XINFER\0\0" and h["format_version"] == 1 and h["header_size"] == 64
        assert h["section_count"] == len(SECTIONS) and h["total_file_size"] == os.path.getsize(p)
        assert r.raw_metadata_json() == meta and r.metadata()["properties"]["hidden_size"] == "5120"
        assert r.list_sections() == [s[0] for s in SECTIONS]
        for name, tag, data in SECTIONS:
            info = r.get_section_info(name)
            assert info.type_tag == tag and info.size == len(data) and info.offset % 64 == 0
            assert info.checksum == (oracle.crc64(data) if data else 0)
            assert r.read_section(name) == data
        assert not r.has_section("nope") and r.get_section_info("nope") is None
        r.validate_checksum()
        raw = p.read_bytes()
        assert r.footer_checksum() == oracle.crc64(raw[:-16]) and raw[-8:] == b"XINFFOOT"


def test_writer_rejects_bad_names():
    w = ArtifactWriter()
    assert w.add_section("a", 0, b"x")
    assert not w.add_section("a", 0, b"y")            # duplicate (writer.cpp:24-29)
    assert not w.add_section("", 0, b"y")             # empty (writer.cpp:21)
    assert not w.add_section("n" * 96, 0, b"y")       # >= 96 bytes
    assert w.add_section("n" * 95, 0, b"y")


def _expect_open_error(path, needle):
    with pytest.raises(ArtifactError) as e:
        ArtifactReader(str(path))
    assert e.value.status == _lib.XINFER_ERR_IO and needle in e.value.message, e.value.message


def test_reader_rejects_malformed(tmp_path):
    p = tmp_path / "a.xinfer"
    _write(p, SECTIONS[:3])
    good = bytearray(p.read_bytes())

    def variant(name, edit):
        b = bytearray(good)
        edit(b)
        q = tmp_path / name
        q.write_bytes(bytes(b))
        return q

    _expect_open_error(tmp_path / "none.xinfer", "Could not open file")
    _expect_open_error(variant("tiny", lambda b: b.__delitem__(slice(70, None))), "smaller than minimum")
    _expect_open_error(variant("magic", lambda b: b.__setitem__(0, ord("Y"))), "Invalid file magic")
    _expect_open_error(variant("ver", lambda b: b.__setitem__(8, 2)), "Unsupported .xinfer format version: 2")
    _expect_open_error(variant("hsz", lambda b: b.__setitem__(12, 65)), "Corrupted header size field")
    _expect_open_error(variant("trunc", lambda b: b.__delitem__(slice(len(b) - 1, None))), "File size mismatch")
    _expect_open_error(variant("foot", lambda b: b.__setitem__(len(b) - 1, 0)), "Invalid footer magic")
    # metadata size pushed past the end of the file
    _expect_open_error(variant("meta", lambda b: b.__setitem__(slice(32, 40), (1 << 40).to_bytes(8, "little"))),
                       "Metadata offset/size points out of bounds")
    # section table size inconsistent with the count
    _expect_open_error(variant("tsz", lambda b: b.__setitem__(slice(48, 56), (129).to_bytes(8, "little"))),
                       "Section table size does not match section count")
    # first section's size pushed past the end
    table = int.from_bytes(good[40:48], "little")
    _expect_open_error(variant("sec", lambda b: b.__setitem__(slice(table + 112, table + 120),
                                                              (1 << 40).to_bytes(8, "little"))),
                       "offset + size points out of bounds")


def test_reader_detects_corruption(tmp_path):
    p = tmp_path / "a.xinfer"
    _write(p, SECTIONS[:4])
    with ArtifactReader(str(p)) as r:
        info = r.get_section_info(SECTIONS[1][0])
    b = bytearray(p.read_bytes())
    b[info.offset + 1000] ^= 0x40
    q = tmp_path / "bad.xinfer"
    q.write_bytes(bytes(b))
    with ArtifactReader(str(q)) as r:  # framing is intact: open succeeds
        with pytest.raises(ArtifactError) as e:
            r.read_section(SECTIONS[1][0])
        assert e.value.status == _lib.XINFER_ERR_CHECKSUM and "Checksum mismatch for section" in e.value.message
        assert r.read_section(SECTIONS[0][0]) == SECTIONS[0][2]   # other sections unaffected
        with pytest.raises(ArtifactError) as e:
            r.validate_checksum()
        assert e.value.status == _lib.XINFER_ERR_CHECKSUM and "checksum mismatch" in e.value.message


def test_golden_reference_written_file():
    """A file written by the reference's ArtifactWriter (fixture): this reader
    reports the same header, section table and footer."""
    exp = json.load(open(os.path.join(GOLDEN, "artifact_ref_small.json")))
    path = os.path.join(GOLDEN, "artifact_ref_small.xinfer")
    raw = open(path, "rb").read()
    with ArtifactReader(path) as r:
        h = r.header()
        for k, v in exp["header"].items():
            assert h[k] == v, k
        assert r.footer_checksum() == int(exp["footer_checksum"], 16) == oracle.crc64(raw[:-16])
        assert r.raw_metadata_json() == exp["metadata"]
        assert r.list_sections() == [s["name"] for s in exp["sections"]]
        for s in exp["sections"]:
            info = r.get_section_info(s["name"])
            assert (info.type_tag, info.flags, info.offset, info.size) == (s["type"], s["flags"], s["offset"], s["size"])
            assert info.checksum == int(s["checksum"], 16)
            data = r.read_section(s["name"])
            assert data == raw[s["offset"]:s["offset"] + s["size"]]
        r.validate_checksum()


# ---------------------------------------------- against the reference build ----

ref_tool = oracle.ref_artifact_tool()
needs_ref = pytest.mark.skipif(ref_tool is None, reason="oracle/_ref/artifact_ref not built (make -C oracle ref)")


def _ref(*args):
    out = subprocess.run([ref_tool, *map(str, args)], check=True, capture_output=True, text=True).stdout
    return out


@needs_ref
def test_same_bytes_as_reference_writer(tmp_path):
    meta = '{"model_name":"x","quant_scheme":"INT4-G128-SYM"}'
    (tmp_path / "meta.json").write_text(meta)
    args = [tmp_path / "ref.xinfer", tmp_path / "meta.json"]
    for i, (name, tag, data) in enumerate(SECTIONS):
        (tmp_path / f"s{i}").write_bytes(data)
        args += [name, int(tag), tmp_path / f"s{i}"]
    assert json.loads(_ref("write", *args))["ok"]
    _write(tmp_path / "ours.xinfer", SECTIONS, meta)
    assert (tmp_path / "ours.xinfer").read_bytes() == (tmp_path / "ref.xinfer").read_bytes()


@needs_ref
def test_reference_reader_accepts_ours_and_agrees_on_corruption(tmp_path):
    p = tmp_path / "ours.xinfer"
    _write(p, SECTIONS)
    d = json.loads(_ref("dump", p))
    assert d["open"] and d["valid"] and all(s["read_ok"] for s in d["sections"])
    with ArtifactReader(str(p)) as r:
        for s in d["sections"]:
            info = r.get_section_info(s["name"])
            assert (info.offset, info.size, info.checksum) == (s["offset"], s["size"], int(s["checksum"], 16))
    assert int(_ref("crc", p), 16) == artifact.crc64_file(str(p))
    b = bytearray(p.read_bytes())
    with ArtifactReader(str(p)) as r:
        off = r.get_section_info(SECTIONS[2][0]).offset
    b[off + 5] ^= 1
    q = tmp_path / "bad.xinfer"
    q.write_bytes(bytes(b))
    d = json.loads(_ref("dump", q))
    ref_bad = {s["name"] for s in d["sections"] if not s["read_ok"]}
    ours_bad = set()
    with ArtifactReader(str(q)) as r:
        for name, _, _ in SECTIONS:
            try:
                r.read_section(name)
            except ArtifactError:
                ours_bad.add(name)
        with pytest.raises(ArtifactError):
            r.validate_checksum()
    assert not d["valid"] and ref_bad == ours_bad == {SECTIONS[2][0]}


@needs_ref
def test_reference_rejects_what_we_reject(tmp_path):
    p = tmp_path / "a.xinfer"
    _write(p, SECTIONS[:2])
    b = bytearray(p.read_bytes())
    b[8] = 7  # version
    q = tmp_path / "v.xinfer"
    q.write_bytes(bytes(b))
    d = json.loads(_ref("dump", q))
    with pytest.raises(ArtifactError) as e:
        ArtifactReader(str(q))
    assert not d["open"] and d["error"] == e.value.message
