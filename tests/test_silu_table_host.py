"""The SwiGLU activation table the build generates (vllm-mach_amd/csrc/silu_table_gen.cpp)
against the oracle's SiLU (oracle/mx_oracle.c mxo_exp, the binary32 sequence of
mxfp8_mlp.py:96): every entry bf16(g / (1 + exp(-g))) for its gate, round to nearest even."""
import re
import subprocess
from pathlib import Path

import numpy as np

import oracle

CSRC = Path(__file__).resolve().parents[1] / "vllm-mach_amd" / "csrc"


def _generated_table(tmp_path):
    exe = tmp_path / "gen"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", f"-I{CSRC}", str(CSRC / "silu_table_gen.cpp"),
                    "-o", str(exe)], check=True)
    out = tmp_path / "silu_table.h"
    subprocess.run([str(exe), str(out)], check=True)
    text = out.read_text()
    body = text[text.index("{") + 1:text.index("}")]
    return np.array([int(v, 16) for v in re.findall(r"0x[0-9a-f]{4}", body)], dtype=np.uint32)


def test_silu_table_matches_oracle(tmp_path):
    src = (CSRC / "silu_math.h").read_text()
    lo = int(re.search(r"kSiluELo = (\d+)", src).group(1))
    hi = int(re.search(r"kSiluEHi = (\d+)", src).group(1))
    span = (hi - lo + 1) << 7
    table = _generated_table(tmp_path)
    assert table.size == 2 * span
    i = np.arange(2 * span, dtype=np.uint32)
    gates = ((lo << 7) + i % span) | np.where(i >= span, 0x8000, 0).astype(np.uint32)
    g = (gates << 16).view(np.float32)
    with np.errstate(over="ignore"):
        act = g / (np.float32(1.0) + oracle.exp_f32(-g))
    u = act.astype(np.float32).view(np.uint32)
    want = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    assert np.array_equal(table, want)
    # the range ends are the documented ones: 2^-24 <= |g| < 256
    assert ((lo << 7) << 16) == np.float32(2.0 ** -24).view(np.uint32)
    assert (((hi + 1) << 7) << 16) == np.float32(256.0).view(np.uint32)
