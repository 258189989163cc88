"""The C-ABI libraries load and export every symbol the headers declare;
host-side argument checking works without a GPU."""
import ctypes
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_libraries_export_every_declared_symbol():
    import rsv
    for lib, hdr in ((rsv.hip_lib(), "rsv_hip.h"), (rsv.host_lib(), "rsv_host.h")):
        names = rsv.declare(lib, os.path.join(ROOT, "include", hdr))
        assert len(names) > 10
        missing = [n for n in names if not hasattr(lib, n)]
        assert not missing, f"{hdr}: missing exports {missing}"


def test_header_declarations_are_parsed_completely():
    import re
    import rsv
    for hdr, lib in (("rsv_hip.h", rsv.hip_lib()), ("rsv_host.h", rsv.host_lib())):
        text = open(os.path.join(ROOT, "include", hdr)).read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        protos = set(re.findall(r"\b(rsv_\w+)\s*\(", text))
        declared = set(rsv.declare(lib, os.path.join(ROOT, "include", hdr)))
        assert protos == declared, protos ^ declared


def test_null_and_missing_arguments_fail_cleanly():
    import rsv
    lib = rsv.hip_lib()
    assert lib.rsv_tensor_create(None, 4, 0, None) != 0
    assert b"null" in lib.rsv_last_error().lower()
    host = rsv.host_lib()
    assert host.rsv_model_build(None, 0, None) != 0
    assert b"null" in host.rsv_host_last_error().lower()
    assert host.rsv_bundle_info(None, None) != 0


def test_no_cpu_fallback_when_library_missing(tmp_path, monkeypatch):
    """The binding refuses to import without the built HIP library."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("rsv_copy", os.path.join(ROOT, "rwkv-rsv_amd", "rsv.py"))
    mod = importlib.util.module_from_spec(spec)
    src = open(os.path.join(ROOT, "rwkv-rsv_amd", "rsv.py")).read()
    src = src.replace('BUILD = os.path.join(HERE, "_build")', f'BUILD = {str(tmp_path)!r}')
    with pytest.raises(Exception, match="not built"):
        exec(compile(src, "rsv_copy", "exec"), mod.__dict__)
