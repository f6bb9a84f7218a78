"""The round-end smoke entry point, run as a GPU test so that it is exercised
with the rest of the suite."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_graft_entry_smoke():
    sys.path.insert(0, ROOT)
    import __graft_entry__
    __graft_entry__.smoke()
