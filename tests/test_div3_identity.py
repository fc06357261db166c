# -*- coding: utf-8 -*-
"""The decoder's ResBlock average ((o1 + o2) + o3) / 3
(``runtime/models/vits.py:2225-2227``) is formed on the GPU by ``div3_rn``
(``csrc/internal.h``): one product and two fused multiply-adds in place of
the IEEE division sequence.  That is bit-identical to the division for every
float32 input; this test checks the identity over all 2^32 bit patterns on
the host (``tests/div3_identity.c``, about 20 s on 8 threads).  The GPU
tests check the kernels that use it through the waveform parity tests."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.timeout(600)
def test_div3_identity_exhaustive(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path / "div3_identity")
    # contraction off: x * r must be rounded before the fused multiply-adds
    base = [gcc, "-O2", "-ffp-contract=off", "-fno-fast-math", os.path.join(HERE, "div3_identity.c"), "-o", exe,
            "-lm"]
    r = subprocess.run(base[:1] + ["-fopenmp"] + base[1:], capture_output=True, text=True)
    if r.returncode != 0:  # no OpenMP runtime: one thread
        r = subprocess.run(base, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=590)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.strip() == "checked 4278190082 mismatches 0"
