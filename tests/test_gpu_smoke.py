"""The driver's round-end smoke check (__graft_entry__.smoke) runs as a GPU
test too, so an API change that breaks it shows up with the other tests."""
import pytest

pytestmark = pytest.mark.gpu


def test_smoke_entry_point():
    import __graft_entry__ as g
    g.smoke()
