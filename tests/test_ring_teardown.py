"""KVRing's destructor must not raise when it runs during interpreter
teardown, after module globals (the library loader, os) have been cleared: a
ring still referenced by a module global is freed through a function bound at
creation.  Runs on the CPU with a stand-in free function."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import sys
sys.path.insert(0, ROOT)
import bmo_jetson_amd.ring as ring_mod

class StandIn(ring_mod.KVRing):
    def __init__(self):  # no device: only the lifetime logic is exercised
        self._h = 1234
        self._free = lambda h: sys.stdout.write("freed %d\n" % h)

KEEP = StandIn()          # freed at interpreter exit, after globals are cleared
ring_mod.lib = None       # as teardown would leave the module
"""


def test_destructor_at_interpreter_exit_is_silent():
    r = subprocess.run([sys.executable, "-c", f"ROOT = {ROOT!r}\n" + SCRIPT],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "Exception ignored" not in r.stderr and "Error" not in r.stderr, r.stderr
    assert "freed 1234" in r.stdout


def test_close_is_idempotent():
    sys.path.insert(0, ROOT)
    import bmo_jetson_amd.ring as ring_mod
    freed = []

    class StandIn(ring_mod.KVRing):
        def __init__(self):
            self._h = 99
            self._free = freed.append

    x = StandIn()
    x.close()
    x.close()
    del x
    assert freed == [99]
