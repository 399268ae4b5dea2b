"""The drop-in boundary's binary layout: include/nve_c_api.h against the
layout measured from the reference's own header (/root/reference/include/
nve_c_api.h:33-835) by tests/golden/c_abi_layout.py, committed as
tests/golden/c_abi_layout.json.  Every struct's size, alignment and field
offsets/sizes, every enumerator's value, the ABI version macros and gcc's
canonical prototype of every function must be identical; the header may
declare nothing the reference's does not.  CPU only (gcc)."""
import json
import os
import re
import shutil
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import c_abi_layout  # noqa: E402

HEADER = os.path.join(ROOT, "include", "nve_c_api.h")

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")


@pytest.fixture(scope="module")
def fixture():
    with open(c_abi_layout.FIXTURE) as f:
        return json.load(f)


def measure(header, fx):
    return c_abi_layout.layout(header, struct_names={k: [f[0] for f in v["fields"]]
                                                     for k, v in fx["structs"].items()},
                               enum_names=list(fx["enums"]))


def differences(got, fx):
    diffs = []
    for name, st in fx["structs"].items():
        if got["structs"].get(name) != st:
            diffs.append(f"struct {name}: {got['structs'].get(name)} != {st}")
    for name, v in fx["enums"].items():
        if got["enums"].get(name) != v:
            diffs.append(f"enum {name}: {got['enums'].get(name)} != {v}")
    if got["macros"] != fx["macros"]:
        diffs.append(f"macros {got['macros']} != {fx['macros']}")
    for name, p in fx["functions"].items():
        if got["functions"].get(name) != p:
            diffs.append(f"function {name}: {got['functions'].get(name)!r} != {p!r}")
    extra = set(got["functions"]) - set(fx["functions"])
    if extra:
        diffs.append(f"functions not in the reference: {sorted(extra)}")
    return diffs


def test_fixture_is_complete(fixture):
    assert len(fixture["structs"]) == 7
    assert len(fixture["functions"]) == 52
    assert fixture["macros"] == {"NVE_C_ABI_VERSION_MAJOR": 1, "NVE_C_ABI_VERSION_MINOR": 0}
    assert fixture["enums"]["NVE_ERROR_OUT_OF_MEMORY"] == 5
    assert fixture["structs"]["nve_gpu_table_config_t"]["size"] == 112


def test_header_layout_matches_the_reference(fixture):
    assert differences(measure(HEADER, fixture), fixture) == []
    # nothing declared beyond the reference's structs and enumerators either
    own = c_abi_layout.layout(HEADER)
    assert set(own["structs"]) == set(fixture["structs"])
    assert set(own["enums"]) == set(fixture["enums"])


@pytest.mark.parametrize("plant", ["swap_fields", "enum_value", "param_type", "extra_function"])
def test_planted_drift_is_caught(tmp_path, fixture, plant):
    """Each kind of drift, planted in a copy of the header, fails the check."""
    text = open(HEADER).read()
    if plant == "swap_fields":
        new = re.sub(r"(\n\s*int\s+disable_uvm_update;[^\n]*)(\n\s*int\s+uvm_cpu_accumulate;[^\n]*)", r"\2\1", text)
        new = re.sub(r"(\n\s*int64_t\s+max_modify_size;)", r"\n  int32_t pad_;\1", new)
    elif plant == "enum_value":
        new = re.sub(r"(NVE_ERROR_OUT_OF_MEMORY\s*=\s*)5", r"\g<1>6", text)
    elif plant == "param_type":
        new = re.sub(r"nve_thread_pool_num_workers\(nve_thread_pool_t pool, int64_t\* out\)",
                     "nve_thread_pool_num_workers(nve_thread_pool_t pool, int32_t* out)", text)
    else:
        new = text.replace("#ifdef __cplusplus\n}", "NVE_C_API nve_status_t nve_extra_call(void);\n#ifdef __cplusplus\n}")
    assert new != text
    h = tmp_path / "nve_c_api.h"
    h.write_text(new)
    assert differences(measure(str(h), fixture), fixture) != []
