"""The host-side code of the library under the CPU sanitizers, fuzzed.

- fastmlx_amd/csrc/fmx_st_parse.cpp (the safetensors header parser, with
  fmxq_status.cpp) is built with g++ -fsanitize=address,undefined and driven by
  tests/fuzz/st_parse_fuzz.cpp with mutants of the reference fixture's blobs
  (compute/testdata/safetensors_header.json, copied to tests/golden/).
- fastmlx_amd/csrc/fmx_shape.cpp (the array-handle layer's shape, broadcast and
  index rules and its buffer-cache bookkeeping) is built the same way, and once
  more with -fsanitize=thread, and driven by tests/fuzz/shape_fuzz.cpp, which
  checks everything the rules accept against brute-force restatements and runs
  the buffer cache from several threads.  This is the counterpart of the
  reference's `go test -race` gate (.github/workflows/ci.yml:34-35) for the
  host logic that needs no GPU.

Any memory error, undefined behaviour, data race, leak or broken invariant fails
the run.
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


def _build_shape_fuzz(tmp_path, sanitize):
    exe = tmp_path / ("shape_fuzz_" + sanitize.replace(",", "_"))
    cmd = ["g++", "-std=c++17", "-g", "-O1", "-fno-omit-frame-pointer",
           f"-fsanitize={sanitize}", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "fuzz", "shape_fuzz.cpp"),
           os.path.join(CSRC, "fmx_shape.cpp"), os.path.join(CSRC, "fmxq_status.cpp"),
           "-o", str(exe), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_shape_rules_fuzz_under_asan(tmp_path):
    exe = _build_shape_fuzz(tmp_path, "address,undefined")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    for seed in ("1", "20260101", "99"):
        r = subprocess.run([str(exe), "20000", seed], capture_output=True, text=True, env=env,
                           timeout=600)
        assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
        assert "buffer cache sequences clean" in r.stdout
        print(r.stdout.strip())


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_shape_rules_and_buffer_cache_under_tsan(tmp_path):
    exe = _build_shape_fuzz(tmp_path, "thread")
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([str(exe), "2000", "5"], capture_output=True, text=True, env=env,
                       timeout=600)
    if r.returncode != 0 and "FATAL: ThreadSanitizer" in r.stderr and "data race" not in r.stderr:
        pytest.skip("ThreadSanitizer cannot run in this environment: " + r.stderr[-300:])
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "buffer cache sequences clean" in r.stdout
