"""The host-side safetensors parser under AddressSanitizer and UBSan, fuzzed.

fastmlx_amd/csrc/fmx_st_parse.cpp (with fmxq_status.cpp) is plain host C++,
so it is built here with g++ -fsanitize=address,undefined.  tests/fuzz/
st_parse_fuzz.cpp then drives it with mutants of the reference fixture's
blobs (compute/testdata/safetensors_header.json, copied to tests/golden/).  Any
memory error, undefined behaviour, leak or broken range invariant fails the
run.
"""
import base64
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "fastmlx_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_safetensors_parser_fuzz_under_asan(tmp_path):
    exe = tmp_path / "st_parse_fuzz"
    cmd = ["g++", "-std=c++17", "-g", "-O1", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "fuzz", "st_parse_fuzz.cpp"),
           os.path.join(CSRC, "fmx_st_parse.cpp"), os.path.join(CSRC, "fmxq_status.cpp"),
           "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    with open(os.path.join(ROOT, "tests", "golden", "safetensors_header.json")) as f:
        cases = json.load(f)["data"]
    seeds = []
    for c in cases:
        p = tmp_path / f"{c['label']}.safetensors"
        p.write_bytes(base64.b64decode(c["blob_b64"]))
        seeds.append(str(p))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), "10000", *seeds], capture_output=True, text=True, env=env,
                       timeout=600)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "mutants parsed" in r.stdout
    print(r.stdout.strip())
