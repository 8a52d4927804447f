"""The decode driver end to end on the GPU (the reference's acceptance run,
README.md:82-89): exit status 0, the acceptance log lines, no error line, the
--oracle check of every step and the every-byte hot-buffer check."""
import os
import re
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(tmp_path, *flags):
    cmd = [sys.executable, "-u", "-m", "kv_offload_proto_amd.xds.xds_decode", "--run-dir", str(tmp_path)] + list(flags)
    print("driver:", " ".join(cmd[3:]), flush=True)
    p = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=240)
    out = p.stdout
    print(out[-3000:], p.stderr[-2000:], flush=True)
    return p.returncode, out


def _accept(rc, out, steps):
    assert rc == 0
    assert "[xds][ERROR]" not in out
    assert re.search(r"\[xds\] pool ready: nodes=\d+ perLayerSegRows=\d+ channels=\d+", out)
    assert re.search(r"\[xds\] prefill export: \d+ rows x \d+ layers = \d+ B in [\d.]+ us", out)
    lines = re.findall(r"\[xds\] step (\d+): layer=(\d+) miss=(\d+) rows in [\d.]+ us \(checked=(\d+)\)", out)
    assert [int(s) for s, *_ in lines] == list(range(steps))
    assert re.search(r"\[xds\] summary: (imported \d+ miss rows, avg [\d.]+ us/row, aggregate [\d.]+ GB/s|no miss)",
                     out)
    assert "[xds] all done" in out
    return lines


def test_driver_reference_defaults_with_oracle(tmp_path):
    """The reference's default shape and stream (8 requests x 64 positions,
    64 slots, prefill 256, 2 layers, 2 segments, 10 steps, seed 42)."""
    rc, out = _run(tmp_path, "--oracle")
    lines = _accept(rc, out, 10)
    assert all(int(m) > 0 and int(c) > 0 for _, _, m, c in lines)
    assert os.path.exists(os.path.join(str(tmp_path), "xds_decode.log"))


def test_driver_shared_slice_fused_state_stream(tmp_path):
    """The reference's shared hot rows (hot stride 0: requests overwrite each
    other and the last position wins), the fused import, a state-driven
    stream, three segments, S = 4 and the fp16 fill."""
    rc, out = _run(tmp_path, "--oracle", "--hot-stride", "0", "--fused", "--stream", "state", "--node-num", "3",
                   "--stripe-rows", "4", "--fill", "fp16", "--steps", "12", "--layers", "3", "--req-num", "6",
                   "--prefill", "300", "--device-buffer-size", "50", "--topk", "40", "--block-dim", "3")
    _accept(rc, out, 12)
