"""Client of the codec JSON-lines driver (mlxl3_amd/exl3_codec), used by the
codec tests: one subprocess per batch of requests, as the reference's harnesses
drive `mlxl3-rs codec`."""

import json
import subprocess
from pathlib import Path

CODEC = Path(__file__).resolve().parent.parent / "mlxl3_amd" / "exl3_codec"


def run(requests, timeout=120):
    text = "".join(json.dumps(r) + "\n" for r in requests)
    res = subprocess.run([str(CODEC), "codec"], input=text, text=True, capture_output=True,
                         check=True, timeout=timeout)
    rows = [json.loads(line) for line in res.stdout.splitlines()]
    assert len(rows) == len(requests), res.stderr
    return rows
