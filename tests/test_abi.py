"""The drop-in boundary without a GPU: both libraries load, every entry point
declared in include/*.h is exported by the library that owns it, the
attestation exports carry the host's ABI fingerprint and the "hip" provider,
and the verified loader refuses a plugin whose attestation does not match.
"""

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(ggml_\w+|openasr_\w+|oa_\w+)\s*\(", re.M)


def declared(header: str) -> list[str]:
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = []
    for m in DECL.finditer(text):
        line = text[m.start():text.find(";", m.start())]
        if "typedef" in line or "(*" in line:
            continue
        names.append(m.group(1))
    return sorted(set(names))


def test_base_exports_every_declared_symbol(ggml):
    lib = C.CDLL(str(ggml.BASE_PATH))
    names = declared("ggml_host.h")
    assert len(names) > 120
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_plugin_exports_every_declared_symbol(ggml):
    lib = C.CDLL(str(ggml.PLUGIN_PATH))
    names = declared("ggml_mi355x.h")
    for required in ("ggml_backend_init", "openasr_ggml_backend_abi_v1", "openasr_ggml_backend_probe_v1",
                     "openasr_ggml_backend_provider_v1"):
        assert required in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_models_library_exports_every_declared_symbol():
    from openasr_amd import decoders as D

    lib = D.lib()
    names = declared("openasr_models.h")
    for required in ("oa_qwen_decode_step", "oa_detect_degenerate_ngram", "oa_classify_quant_tensor_role",
                     "oa_whisper_decode_step"):
        assert required in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_plugin_imports_ggml_base_not_registry(ggml):
    import subprocess
    out = subprocess.run(["readelf", "-d", str(ggml.PLUGIN_PATH)], capture_output=True, text=True).stdout
    needed = re.findall(r"\(NEEDED\).*\[(.*)\]", out)
    assert "libggml-base.so" in needed
    assert not any(n.startswith("libggml.so") for n in needed)


def test_attestation_strings(ggml):
    lib = C.CDLL(str(ggml.PLUGIN_PATH))
    lib.openasr_ggml_backend_abi_v1.restype = C.c_char_p
    lib.openasr_ggml_backend_provider_v1.restype = C.c_char_p
    assert lib.openasr_ggml_backend_provider_v1() == b"hip"
    assert lib.openasr_ggml_backend_abi_v1() == ggml.base().ggml_backend_host_abi_fingerprint()
    from openasr_amd.build import host_abi_fingerprint
    assert lib.openasr_ggml_backend_abi_v1().decode() == host_abi_fingerprint()


def test_verified_loader_rejects_wrong_attestation(ggml):
    lib = ggml.base()
    path = str(ggml.PLUGIN_PATH).encode()
    assert not lib.ggml_backend_load_verified_v3_utf8(path, None, 0, b"0" * 64, b"hip", b"gfx950", b"")
    fp = lib.ggml_backend_host_abi_fingerprint()
    assert not lib.ggml_backend_load_verified_v3_utf8(path, None, 0, fp, b"cuda", b"gfx950", b"")
    assert not lib.ggml_backend_load_verified_v3_utf8(path, None, 0, fp, b"hip", b"gfx1200", b"")
    assert not lib.ggml_backend_load_verified_v3_utf8(b"/nonexistent/plugin.so", None, 0, fp, b"hip", b"", b"")


MEM_STRUCTS = {
    "mem_domain_id": "ggml_backend_memory_domain_id_v1",
    "mem_domain": "ggml_backend_memory_domain_v1",
    "mem_request": "ggml_backend_memory_request_v1",
    "mem_claim": "ggml_backend_memory_claim_v1",
    "mem_quote": "ggml_backend_memory_quote_v1",
    "mem_stats": "ggml_backend_memory_stats_v1",
    "mem_quarantine": "ggml_backend_memory_quarantine_v1",
    "mem_api": "ggml_backend_memory_api_v1",
}


def test_memory_abi_layouts_match_header(ggml, tmp_path):
    """every field offset and struct size of include/ggml_backend_memory.h
    (compiled by gcc) equals the ctypes mirror the tests drive it with"""
    import subprocess
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "ggml_backend_memory.h"', "int main(void) {"]
    for py, c in MEM_STRUCTS.items():
        lines.append(f'printf("{py} %zu\\n", sizeof({c}));')
        for fname, _ in getattr(ggml, py)._fields_:
            lines.append(f'printf("{py}.{fname} %zu\\n", offsetof({c}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    for py in MEM_STRUCTS:
        cls = getattr(ggml, py)
        assert int(got[py]) == C.sizeof(cls), py
        for fname, _ in cls._fields_:
            assert int(got[f"{py}.{fname}"]) == getattr(cls, fname).offset, (py, fname)


def test_memory_abi_table_without_a_device(ggml):
    """the registry proc and the direct export give the same v1 table with
    every entry set (the host's acceptance test, backend_memory.rs:174-184)"""
    lib = C.CDLL(str(ggml.PLUGIN_PATH))
    assert not [n for n in declared("ggml_backend_memory.h") if not hasattr(lib, n)]
    lib.ggml_backend_init.restype = C.c_void_p
    reg = lib.ggml_backend_init()
    assert reg
    proc = ggml.base().ggml_backend_reg_get_proc_address(reg, b"ggml_backend_memory_get_api_v1")
    lib.ggml_backend_memory_get_api_v1.restype = C.c_void_p
    assert proc and C.cast(proc, C.c_void_p).value == C.cast(lib.ggml_backend_memory_get_api_v1, C.c_void_p).value
    api = ggml.MEM_API_GET(proc)().contents
    assert api.struct_size == C.sizeof(ggml.mem_api) and api.abi_version == 1
    for f in ("get_domains", "quote", "reserve_private", "get_stats", "trim", "quarantine"):
        assert getattr(api, f), f
    # calls on handles that are not this plugin's fail instead of crashing
    n = C.c_uint32(0)
    assert api.get_domains(None, None, C.byref(n)) != 0
    assert api.get_stats(None, None, None, C.byref(n)) != 0
    assert api.trim(None, 0) != 0
