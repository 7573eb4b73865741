"""Client of the codec JSON-lines driver (mlxl3_amd/exl3_codec), used by the
codec tests: one subprocess per batch of requests, as the reference's harnesses
drive `mlxl3-rs codec`."""

import json
import os
import subprocess
from pathlib import Path

# EXL3_CODEC selects another build of the driver (the sanitizer build of
# mlxl3_amd/sanitize.py)
CODEC = Path(os.environ.get("EXL3_CODEC")
             or Path(__file__).resolve().parent.parent / "mlxl3_amd" / "exl3_codec")


def run(requests, timeout=120):
    text = "".join(json.dumps(r) + "\n" for r in requests)
    res = subprocess.run([str(CODEC), "codec"], input=text, text=True, capture_output=True,
                         check=True, timeout=timeout)
    rows = [json.loads(line) for line in res.stdout.splitlines()]
    assert len(rows) == len(requests), res.stderr
    return rows
