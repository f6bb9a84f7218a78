"""The checkpoint store reader (qwen-3-ocho_amd/csrc/qfm_store.cpp) on
corrupted inputs, built for the host with AddressSanitizer and
UndefinedBehaviorSanitizer: safetensors shards truncated, header lengths and
header bytes overwritten, JSON offsets / shapes / dtypes replaced by
out-of-range values, manifest.bin truncated or overwritten, shards.txt
pointing at missing or overlong paths. Every case must either open (and then
every entry's bytes lie inside its mapped shard) or be rejected, with no
sanitizer report and no leak. The reference reader these formats come from is
ocho/amd_server/qwenflash.h:12-39 (manifest records) and the safetensors
header layout it parses."""
import json
import os
import random
import shutil
import struct
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import make_store as ms   # noqa: E402


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    d = tmp_path_factory.mktemp("storefuzz")
    exe = str(d / "harness")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + os.path.join(ROOT, "include"), "-o", exe,
           os.path.join(ROOT, "tests", "store_fuzz_harness.cpp"), os.path.join(ROOT, "qwen-3-ocho_amd", "csrc", "qfm_store.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "hip_runtime.h" in r.stderr:
        pytest.skip("HIP headers not available for a host build")
    assert r.returncode == 0, r.stderr[-2000:]
    return exe, d


def _mutate(d, rng):
    sts = sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(".safetensors"))
    st = rng.choice(sts)
    kind = rng.choice(["trunc_st", "flip_hdr", "flip_len", "big_len", "json", "trunc_manifest", "flip_manifest",
                       "shards_txt"])
    b = bytearray(open(st, "rb").read())
    n = struct.unpack("<Q", b[:8])[0]
    if kind == "trunc_st":
        open(st, "r+b").truncate(rng.randrange(0, len(b)))
    elif kind == "flip_hdr":
        for _ in range(rng.randint(1, 8)):
            b[rng.randrange(8, 8 + n)] = rng.randrange(256)
        open(st, "wb").write(b)
    elif kind == "flip_len":
        b[rng.randrange(8)] = rng.randrange(256)
        open(st, "wb").write(b)
    elif kind == "big_len":
        b[:8] = struct.pack("<Q", rng.choice([0, 1, 2 ** 40, 2 ** 63, len(b) - 8, len(b)]))
        open(st, "wb").write(b)
    elif kind == "json":
        h = json.loads(b[8:8 + n])
        k = rng.choice([k for k in h if k != "__metadata__"])
        m = rng.choice(["offsets", "shape", "dtype", "huge"])
        if m == "offsets":
            h[k]["data_offsets"] = [rng.randrange(-5, 10 ** 7), rng.randrange(-5, 10 ** 7)]
        elif m == "shape":
            h[k]["shape"] = [rng.randrange(0, 10 ** 5) for _ in range(rng.randint(0, 6))]
        elif m == "dtype":
            h[k]["dtype"] = rng.choice(["F33", "", "BF16x", "I8"])
        else:
            h[k]["data_offsets"] = [2 ** 63, 2 ** 64 - 1]
        hb = json.dumps(h).encode()
        open(st, "wb").write(struct.pack("<Q", len(hb)) + hb + b[8 + n:])
    elif kind == "trunc_manifest":
        m = os.path.join(d, "manifest.bin")
        open(m, "r+b").truncate(rng.randrange(0, os.path.getsize(m)))
    elif kind == "flip_manifest":
        m = os.path.join(d, "manifest.bin")
        mb = bytearray(open(m, "rb").read())
        for _ in range(rng.randint(1, 16)):
            mb[rng.randrange(len(mb))] = rng.randrange(256)
        open(m, "wb").write(mb)
    else:
        open(os.path.join(d, "shards.txt"), "w").write(
            rng.choice(["", "nonexistent.safetensors\n", "../../etc/passwd\n", "x" * 5000 + "\n"]))
    return st


def test_store_reader_survives_corrupted_inputs(harness):
    exe, tmp = harness
    base = str(tmp / "base")
    ms.synthetic_layer(base, 64, 32, 4, 0, 7, shards=2)
    ms.manifest_from_safetensors(base, sorted(os.path.join(base, f) for f in os.listdir(base)
                                              if f.endswith(".safetensors")))
    rng = random.Random(1)
    cases = [base, os.path.join(base, sorted(f for f in os.listdir(base) if f.endswith(".safetensors"))[0])]
    for i in range(160):
        d = str(tmp / f"c{i}")
        shutil.copytree(base, d)
        cases += [d, _mutate(d, rng)]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe] + cases, capture_output=True, text=True, env=env)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    opened, rejected = (int(v) for v in r.stdout.split()[1::2])
    assert opened >= 2 and rejected > 0 and opened + rejected == len(cases)
