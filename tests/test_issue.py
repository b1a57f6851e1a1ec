"""The compiled issue loop (madi_amd/libmadi_issue.so): it exports its one
entry point, and a replayed call fails the way the direct call does (here a
shape the library refuses before touching a device: MADI_ERR_SHAPE, with the
index of the failing call)."""
import pytest

import madi_amd
from madi_amd import issue
from madi_amd.q8 import Q8

FAKE = 0x100000


def test_issue_library_loads_and_exports():
    L = issue.lib()
    assert hasattr(L, "madi_issue_run")


def test_replayed_call_reports_the_library_error():
    lst = issue.IssueList()
    w = Q8(FAKE, FAKE)
    lst.kGemvQ8(FAKE, FAKE, w, 1280, 96)   # k % 64: refused before the device is needed
    lst.kGemvQ8(FAKE, FAKE, w, 1280, 96)
    assert len(lst) == 2
    with pytest.raises(madi_amd.MadiError) as e:
        lst.run(3)
    assert e.value.code == -5
    assert "call 0" in str(e.value)


def test_empty_list_runs():
    issue.IssueList().run(5)
