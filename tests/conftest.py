# -*- coding: utf-8 -*-
"""Shared pytest setup: import paths, the ``gpu`` marker and fixtures."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "rvc-vulkan_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP backend)")


def rel_l2(a, b):
    """||a-b||_2 / ||b||_2, the per-op error measure of the reference engine
    self-test (engine/test_ffi.py:103-105)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.linalg.norm((a - b).ravel())
    n = np.linalg.norm(b.ravel())
    return float(d / n) if n > 0 else float(d)


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN
