"""libggml-hip.so as a dlopen backend module: the entry points and registry
object that llama.rust's ggml_backend_load reads (crates/ggml/src/backend.rs:1354-1420,
sysffi.rs:118-171).  CPU only: on a host without a gfx950 device the module
scores 0 and lists no devices; the loader's refusal paths are exercised with
small stub modules, as the reference's own dlopen test does
(backend.rs:2460-2560)."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

import backend_reg as BR
import ghip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header, prefix):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", src)))


def test_module_exports_declared_entry_points():
    names = declared("ggml_hip_reg.h", "ggml_backend_")
    assert names == ["ggml_backend_init", "ggml_backend_score"]
    h = ctypes.CDLL(BR.MODULE_PATH)
    assert all(hasattr(h, n) for n in names)


def test_registry_object():
    b = BR.init_unscored()
    assert b.api_version == BR.GGML_BACKEND_API_VERSION == 2
    assert b.name == "HIP"
    # a second init returns the same static object (the device list is fixed)
    again = BR.init_unscored()
    assert ctypes.addressof(again._reg.contents) == ctypes.addressof(b._reg.contents)


def test_proc_addresses_are_the_ghip_entry_points():
    b = BR.init_unscored()
    lib = ghip.lib()
    names = declared("ghip.h", "ghip_")
    assert "ghip_mul_mat" in names and "ghip_flash_attn_ext" in names
    for n in names:
        want = ctypes.cast(getattr(lib, n), ctypes.c_void_p).value
        assert b.proc_address(n) == want, n
    assert b.proc_address("ggml_backend_init") == 0
    assert b.proc_address("ghip_nosuch") == 0


def test_score_gates_load():
    h = ctypes.CDLL(BR.MODULE_PATH)
    h.ggml_backend_score.restype = ctypes.c_int
    score = h.ggml_backend_score()
    assert score >= 0
    if score == 0:  # no gfx950 device visible (this container)
        with pytest.raises(BR.LoadError, match="not supported on this system"):
            BR.load()
        assert BR.init_unscored().devices() == []
    else:
        b = BR.load()
        assert len(b.devices()) >= 1


STUB = r"""
#include <stddef.h>
typedef const char *(*name_fn)(const void *);
typedef struct { name_fn get_name; size_t (*count)(const void *); void *(*dev)(const void *, size_t);
                 void *(*proc)(const void *, const char *); } reg_i;
typedef struct { int api_version; reg_i iface; void *context; } reg_t;
static const char *nm(const void *r) { (void)r; return "STUB"; }
static size_t cnt(const void *r) { (void)r; return 0; }
static void *dv(const void *r, size_t i) { (void)r; (void)i; return NULL; }
static reg_t the_reg = { API, { nm, cnt, dv, NULL }, NULL };
SCORE
INIT
"""


def stub(tmp_path, name, api=2, score=None, init="ok"):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = STUB.replace("API", str(api))
    src = src.replace("SCORE", "" if score is None else f"int ggml_backend_score(void) {{ return {score}; }}")
    src = src.replace("INIT", {"ok": "void *ggml_backend_init(void) { return &the_reg; }",
                               "null": "void *ggml_backend_init(void) { return NULL; }",
                               "none": ""}[init])
    c = tmp_path / (name + ".c")
    so = tmp_path / (name + ".so")
    c.write_text(src)
    subprocess.run([cc, "-shared", "-fPIC", "-o", str(so), str(c)], check=True)
    return str(so)


def test_loader_refusals(tmp_path):
    """backend.rs:1354-1410: every refusal of ggml_backend_load, and a good module"""
    with pytest.raises(BR.LoadError, match="failed to load"):
        BR.load(str(tmp_path / "libggml-nosuch.so"))
    with pytest.raises(BR.LoadError, match="not supported"):
        BR.load(stub(tmp_path, "zero", score=0))
    with pytest.raises(BR.LoadError, match="failed to find ggml_backend_init"):
        BR.load(stub(tmp_path, "noinit", init="none"))
    with pytest.raises(BR.LoadError, match="returned NULL"):
        BR.load(stub(tmp_path, "nullinit", init="null"))
    with pytest.raises(BR.LoadError, match=r"incompatible API version \(backend: 3, current: 2\)"):
        BR.load(stub(tmp_path, "api3", api=3))
    ok = BR.load(stub(tmp_path, "good", score=5))
    assert ok.name == "STUB" and ok.devices() == []
