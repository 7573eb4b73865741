"""Collect the reference's golden vectors for the EXL3 path into tests/golden/.

Run in the build container (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py [/root/reference]

Everything written here is data -- inputs and expected outputs the reference's
own tests and fixtures hold -- verified against the checksums the reference
records for them:

* quantizer/   tests/fixtures/native-quantizer/oracle-{K}-{cb}-{packed,states,decoded}
               (K = 2..8, cb = 0..2, 4 tiles each; sha256 from reference.json).  Used by
               tests/test_native_quantizer.py:299-336.  The only 3INST vectors.
* real_tiles/  docs/native-coverage/baselines/exl3/{flash,qwen-dense,qwen-moe,lfm-moe}.json
               (3 real checkpoint tiles each: packed, states, f16 bits, and the
               byte offset of each tile in its shard).  Used by
               native/tests/contracts.rs:617-669.
* hadamard/    tests/fixtures/native-converter-host/hadamard.{npz,json} (MLX 0.32.2 f32
               hadamard_transform outputs; sha256 in hadamard.json).  Used by
               tests/test_native_transforms.py:95-110.
* tables.json  the 1021 MUL1 f16 values listed in native/shaders/ar33_codeword_table.metal
               and the 256 positions listed in native/shaders/flash_reference_reduction.h
               (numbers only).
"""

from __future__ import annotations

import hashlib
import json
import re
import shutil
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent


def sha256(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def main(ref: Path) -> None:
    q_src = ref / "tests/fixtures/native-quantizer"
    q_dst = OUT / "quantizer"
    q_dst.mkdir(exist_ok=True)
    report = json.loads((q_src / "reference.json").read_text())
    for name, digest in report["files"].items():
        if not name.startswith("oracle-"):
            continue
        src = q_src / name
        assert sha256(src) == digest, name
        shutil.copyfile(src, q_dst / name)
    (q_dst / "checksums.json").write_text(
        json.dumps({k: v for k, v in report["files"].items() if k.startswith("oracle-")},
                   indent=1, sort_keys=True)
    )

    t_src = ref / "docs/native-coverage/baselines/exl3"
    t_dst = OUT / "real_tiles"
    t_dst.mkdir(exist_ok=True)
    for name in ("flash", "qwen-dense", "qwen-moe", "lfm-moe"):
        data = json.loads((t_src / f"{name}.json").read_text())
        keep = {
            k: data[k]
            for k in ("checkpoint", "shard", "header_sha256", "tensor", "dtype", "shape", "k", "mode")
        }
        keep["tiles"] = [
            {k: t[k] for k in ("tile", "shard_offset_bytes", "packed", "states", "f16_bits")}
            for t in data["tiles"]
        ]
        (t_dst / f"{name}.json").write_text(json.dumps(keep))

    h_src = ref / "tests/fixtures/native-converter-host"
    h_dst = OUT / "hadamard"
    h_dst.mkdir(exist_ok=True)
    meta = json.loads((h_src / "hadamard.json").read_text())
    assert sha256(h_src / "hadamard.npz") == meta["sha256"]
    shutil.copyfile(h_src / "hadamard.npz", h_dst / "hadamard.npz")
    shutil.copyfile(h_src / "hadamard.json", h_dst / "hadamard.json")

    shaders = ref / "native/shaders"
    table_text = (shaders / "ar33_codeword_table.metal").read_text()
    body = table_text[table_text.index("{") + 1 : table_text.index("}")]
    mul1 = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", body)]
    assert len(mul1) == 1021
    pos_text = (shaders / "flash_reference_reduction.h").read_text()
    positions = [int(v) for v in pos_text[pos_text.index("{") + 1 : pos_text.index("}")].split(",")]
    assert len(positions) == 256
    (OUT / "tables.json").write_text(
        json.dumps({"mul1_sum_to_f16": mul1, "reference_positions": positions})
    )
    print("golden fixtures written to", OUT)


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
