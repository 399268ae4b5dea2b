"""The leveled logger (include/logging.hpp:34-203 in the reference): the level
comes from NVE_LOG_LEVEL and the C ABI, messages at or below it are written
(errors to stderr, the rest to stdout), others are not formatted at all.  Runs
in subprocesses so that the environment variable is read afresh."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SNIPPET = r"""
import ctypes, sys
sys.path.insert(0, {pkg!r})
from pynve import _lib
L = _lib.load()
lvl = ctypes.c_int32()
assert L.nve_amd_get_log_level(ctypes.byref(lvl)) == 0
print("LEVEL", lvl.value, flush=True)
# a rejected argument is logged at the info level
rc = L.nve_amd_set_log_level(-5)
print("RC", rc, flush=True)
"""


def run(env_level):
    env = dict(os.environ)
    env.pop("NVE_LOG_LEVEL", None)
    if env_level is not None:
        env["NVE_LOG_LEVEL"] = env_level
    code = SNIPPET.format(pkg=os.path.join(ROOT, "nv-embedding-cache_amd"))
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert p.returncode == 0, p.stderr
    return p.stdout, p.stderr


@pytest.mark.parametrize("name,value", [("CRITICAL", 0), ("ERROR", 10), ("WARNING", 20), ("PERF", 30),
                                        ("INFO", 40), ("VERBOSE", 100)])
def test_env_level_names(name, value):
    out, _ = run(name)
    assert f"LEVEL {value}" in out


def test_default_is_warning_and_info_messages_are_filtered():
    out, err = run(None)
    assert "LEVEL 20" in out and "RC 1" in out
    assert "[NVE" not in out and "[NVE" not in err


def test_info_level_writes_rejected_arguments_to_stdout():
    out, err = run("INFO")
    assert "RC 1" in out
    line = [s for s in out.splitlines() if s.startswith("[NVE")]
    assert line and "[I] status 1: log level must not be negative" in line[0]
    assert "[NVE" not in err


def test_unknown_name_warns_and_keeps_warning():
    out, err = run("LOUD")
    assert "LEVEL 20" in out
    assert "NVE_LOG_LEVEL=LOUD" in err


def test_set_and_get_through_the_c_abi():
    import ctypes
    sys.path.insert(0, os.path.join(ROOT, "nv-embedding-cache_amd"))
    from pynve import _lib
    L = _lib.load()
    old = ctypes.c_int32()
    assert L.nve_amd_get_log_level(ctypes.byref(old)) == 0
    try:
        assert L.nve_amd_set_log_level(40) == 0
        got = ctypes.c_int32()
        assert L.nve_amd_get_log_level(ctypes.byref(got)) == 0 and got.value == 40
        assert L.nve_amd_get_log_level(None) != 0
    finally:
        L.nve_amd_set_log_level(old.value)
