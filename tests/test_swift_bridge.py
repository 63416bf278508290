"""The Swift HIPBridge module (minirun-app_amd/swift) as source: every
function include/minirun_hip.h declares is called by a wrapper, the module
map names the header, and each wrapper file cites the reference interface
it replaces.  There is no Swift toolchain here, so the check is textual; the
C-level ABI test (test_abi.py) compiles the same header as C."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SWIFT = os.path.join(ROOT, "minirun-app_amd", "swift")


def declared():
    text = open(os.path.join(ROOT, "include", "minirun_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mr_[a-z0-9_]+)\s*\(", text)))


def swift_sources():
    d = os.path.join(SWIFT, "Sources", "HIPBridge")
    return {f: open(os.path.join(d, f)).read() for f in sorted(os.listdir(d)) if f.endswith(".swift")}


def test_every_entry_point_has_a_wrapper():
    calls = set()
    for text in swift_sources().values():
        code = re.sub(r"//.*", "", text)
        calls |= set(re.findall(r"\b(mr_[a-z0-9_]+)\s*\(", code))
    missing = [n for n in declared() if n not in calls]
    assert not missing, f"declared in the header, no Swift wrapper calls them: {missing}"
    text = open(os.path.join(ROOT, "include", "minirun_hip.h")).read()
    types = set(re.findall(r"}\s*(mr_[a-z0-9_]+)\s*;", text))  # struct initialisers, not calls
    unknown = sorted(calls - set(declared()) - types)
    assert not unknown, f"Swift calls functions the header does not declare: {unknown}"


def test_module_map_and_package():
    mm = open(os.path.join(SWIFT, "Sources", "CMinirunHIP", "module.modulemap")).read()
    m = re.search(r'header\s+"([^"]+)"', mm)
    assert m, mm
    hdr = os.path.normpath(os.path.join(SWIFT, "Sources", "CMinirunHIP", m.group(1)))
    assert hdr == os.path.join(ROOT, "include", "minirun_hip.h")
    assert 'link "minirun_hip"' in mm
    pkg = open(os.path.join(SWIFT, "Package.swift")).read()
    assert ".systemLibrary(name: \"CMinirunHIP\"" in pkg and ".target(name: \"HIPBridge\"" in pkg


def test_wrappers_cite_the_reference():
    for name, text in swift_sources().items():
        if name == "HIPTypes.swift":
            continue
        assert re.search(r"\w+\.swift:\d+", text), f"{name} cites no reference file:line"
    # each public wrapper function carries a doc comment naming what it replaces
    for name, text in swift_sources().items():
        for m in re.finditer(r"\n((?:///.*\n)*)(?:@discardableResult\n)?public func (\w+)", text):
            assert m.group(1).strip(), f"{name}: {m.group(2)} has no doc comment"


def test_swift_field_names_match_the_header_structs():
    # the struct fields the wrappers set exist in the C structs they fill
    text = open(os.path.join(ROOT, "include", "minirun_hip.h")).read()
    fields = set(re.findall(r"\b([a-z_][a-z0-9_]*)\s*[;,]", text))
    for name, src in swift_sources().items():
        for f in re.findall(r"\ba\.([a-z_][a-z0-9_]*)\s*=", src):
            assert f in fields, f"{name}: a.{f} is not a field of the header's structs"
