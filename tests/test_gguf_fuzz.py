"""The GGUF reader on malformed input, host code under AddressSanitizer / UndefinedBehaviorSanitizer (no GPU).

A tiny model file of the reference's layout is mutated (bit flips, truncations, 4- and 8-byte overwrites with
boundary values, deleted runs) in its header region; the reader, built with g++ and the sanitizers beside a small
driver, must parse or refuse every variant without a sanitizer report.  Files the reader accepts have their tensors'
first and last bytes read back, so a tensor extent past the mapping would be reported."""

import os
import random
import shutil
import struct
import subprocess

import pytest

import model_synth as ms

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "..", "faie2-flashnext_amd", "csrc", "gguf.cpp")


def _mutate(raw, rng, hdr):
    b = bytearray(raw)
    kind = rng.randrange(5)
    if kind == 0:
        for _ in range(rng.randrange(1, 8)):
            b[rng.randrange(hdr)] ^= 1 << rng.randrange(8)
    elif kind == 1:
        b = b[: rng.randrange(len(b))]
    elif kind == 2:
        o = rng.randrange(hdr - 8)
        b[o:o + 8] = struct.pack("<Q", rng.choice([0, 1, 2**31, 2**32 - 1, 2**63, 2**64 - 1, rng.getrandbits(64)]))
    elif kind == 3:
        o = rng.randrange(hdr - 4)
        b[o:o + 4] = struct.pack("<I", rng.choice([0, 1, 12, 30, 255, 2**31, 2**32 - 1, rng.getrandbits(32)]))
    else:
        o = rng.randrange(hdr)
        del b[o:o + rng.randrange(1, 64)]
    return bytes(b)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_gguf_reader_survives_mutated_files_under_sanitizers(tmp_path):
    exe = str(tmp_path / "gguf_fuzz")
    r = subprocess.run(["g++", "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-fno-omit-frame-pointer", SRC, os.path.join(HERE, "gguf_fuzz_driver.cpp"), "-o", exe],
                       capture_output=True, text=True)
    if r.returncode and "sanitize" in r.stderr and "cannot find" in r.stderr:
        pytest.skip("sanitizer runtime not installed")
    assert r.returncode == 0, r.stderr[-2000:]
    base = str(tmp_path / "base.gguf")
    ms.write_model(base, ms.TINY_DIMS, seed=3)
    raw = open(base, "rb").read()
    hdr = min(len(raw), 40000)
    rng = random.Random(2024)
    parsed = refused = 0
    for batch in range(6):
        paths = []
        for i in range(50):
            p = str(tmp_path / f"m{i}.gguf")
            open(p, "wb").write(_mutate(raw, rng, hdr))
            paths.append(p)
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
        out = subprocess.run([exe, base] + paths, capture_output=True, text=True, env=env, timeout=300)
        assert out.returncode == 0, (batch, out.stdout[-500:], out.stderr[-3000:])
        assert "runtime error" not in out.stderr and "AddressSanitizer" not in out.stderr, out.stderr[-3000:]
        words = out.stdout.split()
        parsed += int(words[1]) - 1
        refused += int(words[3])
    for i in range(50):
        os.remove(str(tmp_path / f"m{i}.gguf"))
    assert parsed + refused == 300
    assert parsed > 0 and refused > 0  # both paths exercised
