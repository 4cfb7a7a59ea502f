"""The JSON-line engine server (mars_amd/mars_engine; protocol of the reference's
src/engine_server.cu:9-14, 242-354): requests that need no graph, on the CPU.
The engine makes no GPU call before its first ADD or LOAD."""
from __future__ import annotations

import json
import subprocess

import pytest

from conftest import ROOT

ENGINE = ROOT / "mars_amd" / "mars_engine"


def run(lines, dim=4):
    p = subprocess.run([str(ENGINE), "--dim", str(dim)], input="\n".join(lines) + "\n", capture_output=True,
                       text=True, timeout=60)
    assert p.returncode == 0, p.stderr
    return [json.loads(x) for x in p.stdout.splitlines()]


@pytest.mark.skipif(not ENGINE.exists(), reason="engine not built")
def test_protocol_without_a_graph():
    out = run([
        '{"cmd":"STATS"}',
        '{"cmd":"QUERY","embedding":[1,0,0,0],"top_k":5}',
        '{"cmd":"QUERY","embedding":[1,0,0],"top_k":5}',
        '{"cmd":"ADD","id":0,"modality":1,"embedding":[1,2],"timestamp":3}',
        '{"cmd":"DELETE","id":3}',
        '{"cmd":"FLY"}',
        '{"cmd":"QUERY", "embedding":[1,0,0,0]',
        'not json',
        '{"cmd":"SAVE","path":"/nonexistent/x.mars"}',
        '{"cmd":"LOAD"}',
        '{"cmd":"SHUTDOWN"}',
        '{"cmd":"STATS"}',                      # after SHUTDOWN: never read
    ])
    assert out[0] == {"n": 0, "edges": 0, "vram_mb": 0.0}
    assert out[1] == {"results": []}
    assert out[2] == {"ok": False, "error": "query embedding dimension mismatch"}
    assert out[3] == {"ok": False, "error": "embedding dimension mismatch"}
    assert out[4] == {"ok": True}
    assert out[5] == {"ok": False, "error": "unknown command"}
    assert out[6] == out[7] == {"ok": False, "error": "malformed JSON"}
    assert out[8] == {"ok": False, "error": "no graph to save"}
    assert out[9] == {"ok": False, "error": "LOAD needs a path"}
    assert out[10] == {"ok": True}
    assert len(out) == 11
