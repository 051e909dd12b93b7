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
