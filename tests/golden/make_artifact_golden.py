"""Writes tests/golden/artifact_ref_small.xinfer and its expected values with
the REFERENCE artifact writer (src/artifact/writer.cpp, built from the
reference sources by `make -C oracle ref` into oracle/_ref/artifact_ref).

The file holds one small INT4-G128 projection (`<name>` + `<name>.scales`,
quantized from a seeded tensor by the oracle's restatement of
convert.py:93-119), an odd-sized tokenizer blob, a chat template and an empty
section.  artifact_ref_small.json records what the reference reader reports
for it (header fields, section table, footer CRC) plus CRC-64 values from the
oracle, so that this build's reader is checked against the reference format
also where the reference tree is absent.

    make -C oracle ref && python tests/golden/make_artifact_golden.py
"""
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from xinfer_amd import synth  # noqa: E402

NAME = "model.layers.0.mlp.down_proj.weight"
N, K = 64, 256
META = ('{"model_name":"Qwen/Qwen3.8-27B","quant_scheme":"INT4-G128-SYM",'
        '"tokenizer_type":"qwen3_8_tiktoken","properties":{"hidden_size":"5120"}}')


def main():
    tool = oracle.ref_artifact_tool()
    if tool is None:
        raise SystemExit("oracle/_ref/artifact_ref is missing: run `make -C oracle ref`")
    rng = np.random.default_rng(20261201)
    w = rng.normal(0.0, 0.02, size=(N, K)).astype(np.float32)
    W, S = oracle.quantize_int4(w)
    tok = bytes(rng.integers(0, 256, 1001, dtype=np.uint8))
    tmpl = b"{% for message in messages %}{{ message['content'] }}{% endfor %}"
    sections = [(NAME, 3, W.tobytes()), (NAME + ".scales", 4, S.tobytes()),
                ("tokenizer.data", 2, tok), ("chat_template.jinja", 5, tmpl), ("empty.blob", 0, b"")]
    out = os.path.join(HERE, "artifact_ref_small.xinfer")
    with tempfile.TemporaryDirectory() as td:
        meta = os.path.join(td, "meta.json")
        open(meta, "w").write(META)
        args = [tool, "write", out, meta]
        for i, (name, tag, data) in enumerate(sections):
            p = os.path.join(td, f"s{i}")
            open(p, "wb").write(data)
            args += [name, str(tag), p]
        subprocess.run(args, check=True, capture_output=True)
    dump = json.loads(subprocess.run([tool, "dump", out], check=True, capture_output=True, text=True).stdout)
    assert dump["open"] and dump["valid"] and all(s["read_ok"] for s in dump["sections"])
    for s, (name, tag, data) in zip(dump["sections"], sections):
        assert s["name"] == name and s["size"] == len(data)
        assert int(s["checksum"], 16) == (oracle.crc64(data) if data else 0)
    expected = {
        "reference": "src/artifact/writer.cpp (ArtifactWriter, raw metadata JSON)",
        "header": dump["header"],
        "footer_checksum": dump["footer_checksum"],
        "metadata": dump["metadata"],
        "sections": [{k: s[k] for k in ("name", "type", "flags", "offset", "size", "checksum")}
                     for s in dump["sections"]],
        "linear": {"name": NAME, "out_features": N, "in_features": K, "group_size": 128},
    }
    with open(os.path.join(HERE, "artifact_ref_small.json"), "w") as f:
        json.dump(expected, f, indent=1)
    print("wrote", out)


if __name__ == "__main__":
    main()
