"""Loader of oracle/_ref: the reference's own HIP kernels for this path,
compiled in place from the reference checkout by oracle/Makefile (`make ref`)
with the library's code-generation flags. Test infrastructure only; absent
where the checkout was not available at build time (the tests then skip)."""
import ctypes as C
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNELS = os.path.join(ROOT, "oracle", "_ref", "libqfm_ref.so")
READER = os.path.join(ROOT, "oracle", "_ref", "libqf_reader_ref.so")
_libs = {}


def _load(path):
    if path not in _libs:
        if not os.path.exists(path):
            pytest.skip(f"{os.path.relpath(path, ROOT)} not built (made by oracle/Makefile `ref` where the "
                        "reference checkout exists)")
        _libs[path] = C.CDLL(path)          # RTLD_LOCAL: its symbols never bind libqfm's
    return _libs[path]


def kernels():
    return _load(KERNELS)


def reader():
    return _load(READER)
