"""Binary layout of a C-ABI header, measured by the C compiler.

`layout(header)` compiles small C programs against the header and returns:
  * structs: for every `typedef struct { ... } name;` its sizeof / alignof and
    each field's offsetof and sizeof;
  * enums: the value of every enumerator;
  * macros: the NVE_C_ABI_VERSION_* values;
  * functions: gcc's own canonical prototype of every `nve_*` function
    (`-aux-info`: parameter types only, names dropped).

Run as a script in a container that holds the reference sources
(/root/reference/include/nve_c_api.h, the interface `include/nve_c_api.h`
must match byte for byte in layout), it writes tests/golden/c_abi_layout.json.
tests/test_c_abi_layout.py measures this build's header the same way and
compares.  The fixture is data measured from the reference's header (sizes,
offsets, values, compiler-canonicalised signatures), not its text.
"""
import json
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "c_abi_layout.json")
REFERENCE_HEADER = "/root/reference/include/nve_c_api.h"


def _preprocessed(header, cc):
    out = subprocess.run([cc, "-E", "-P", "-x", "c", header], check=True, capture_output=True, text=True)
    return out.stdout


def _structs(pre):
    found = {}
    for body, name in re.findall(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", pre, flags=re.S):
        if not name.startswith("nve_"):
            continue  # the system headers' own (max_align_t)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            m = re.search(r"(\w+)\s*(\[[^\]]*\])?\s*$", decl)
            fields.append(m.group(1))
        found[name] = fields
    return found


def _enumerators(pre):
    names = []
    for body in re.findall(r"enum\s*\w*\s*\{(.*?)\}", pre, flags=re.S):
        for item in body.split(","):
            item = item.strip()
            name = re.match(r"(\w+)", item).group(1) if item else ""
            if name.startswith("NVE_"):
                names.append(name)
    return names


def _run(src, header, cc, workdir):
    c = os.path.join(workdir, "probe.c")
    exe = os.path.join(workdir, "probe")
    with open(c, "w") as f:
        f.write(src)
    subprocess.run([cc, "-std=c11", "-Wall", "-I", os.path.dirname(os.path.abspath(header)), "-o", exe, c],
                   check=True, capture_output=True, text=True)
    return json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)


def _functions(header, cc, workdir):
    aux = os.path.join(workdir, "aux.txt")
    subprocess.run([cc, "-std=c11", "-fsyntax-only", "-x", "c", "-aux-info", aux, header], check=True,
                   capture_output=True, text=True)
    protos = {}
    for line in open(aux):
        line = re.sub(r"/\*.*?\*/", "", line).strip()
        m = re.search(r"\b(nve_\w+)\s*\(", line)
        if m:
            protos[m.group(1)] = re.sub(r"\s+", " ", line.replace("extern ", "", 1)).rstrip(";").strip()
    return protos


def layout(header, cc="gcc", struct_names=None, enum_names=None):
    """Layout of `header`.  With struct_names / enum_names (a fixture's), those
    are measured, so a field or enumerator missing from `header` fails to
    compile rather than going unchecked."""
    pre = _preprocessed(header, cc)
    structs = _structs(pre) if struct_names is None else struct_names
    enums = _enumerators(pre) if enum_names is None else enum_names
    lines = ["#include <stdio.h>", "#include <stddef.h>", "#include <stdalign.h>",
             f'#include "{os.path.basename(header)}"', "int main(void) {", 'printf("{\\"structs\\": {");']
    for si, (name, fields) in enumerate(structs.items()):
        lines.append(f'printf("%s\\"{name}\\": {{\\"size\\": %zu, \\"align\\": %zu, \\"fields\\": [", '
                     f'"{"," if si else ""}", sizeof({name}), alignof({name}));')
        for fi, f in enumerate(fields):
            lines.append(f'printf("%s[\\"{f}\\", %zu, %zu]", "{"," if fi else ""}", offsetof({name}, {f}), '
                         f"sizeof((({name}*)0)->{f}));")
        lines.append('printf("]}");')
    lines.append('printf("}, \\"enums\\": {");')
    for ei, e in enumerate(enums):
        lines.append(f'printf("%s\\"{e}\\": %lld", "{"," if ei else ""}", (long long){e});')
    lines.append('printf("}, \\"macros\\": {\\"NVE_C_ABI_VERSION_MAJOR\\": %d, \\"NVE_C_ABI_VERSION_MINOR\\": %d}}",'
                 " (int)NVE_C_ABI_VERSION_MAJOR, (int)NVE_C_ABI_VERSION_MINOR);")
    lines += ["return 0;", "}"]
    with tempfile.TemporaryDirectory() as d:
        out = _run("\n".join(lines) + "\n", header, cc, d)
        out["functions"] = _functions(header, cc, d)
    # fields as lists of [name, offset, size]; keep the struct order of the header
    out["struct_order"] = list(structs)
    return out


def main():
    header = sys.argv[1] if len(sys.argv) > 1 else REFERENCE_HEADER
    data = layout(header)
    with open(FIXTURE, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"{FIXTURE}: {len(data['structs'])} structs, {len(data['enums'])} enumerators, "
          f"{len(data['functions'])} functions")


if __name__ == "__main__":
    main()
