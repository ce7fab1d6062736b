"""The code-object disk cache without a GPU (reference: newt/runtime/jit.py:50-65,
where CompiledKernel keys sha256(source + arch + version), loads the cached
image on a hit and writes image + source on a miss).

A kernel is compiled through JITFunction's own compile path with the module
loader replaced by a stand-in (loading needs a GPU); hipRTC runs for real.
Checked: a miss writes <key>.hsaco, <key>.sha256 and <key>.hip; a fresh
JITFunction is served from disk with the compiler disabled; the key changes
with the backend version and the compile options; a corrupted, truncated or
digest-less image is detected on the host and rebuilt."""

import os

import pytest

import newt_amd.language as nl
from newt_amd.compiler import types as tp
from newt_amd.runtime import hip
from newt_amd.runtime import jit as J


def _kernel(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    m = offs < n
    nl.store(o_ptr + offs, nl.load(x_ptr + offs, mask=m) * 3.0, mask=m)


class _LoadedModule:
    """Stands in for hip.Kernel (module load needs a GPU): keeps the image."""

    def __init__(self, code, name, lds):
        assert code[:4] == b"\x7fELF"
        self.code, self.name = code, name


@pytest.fixture
def cache(tmp_path, monkeypatch):
    monkeypatch.setenv("NEWT_CACHE_DIR", str(tmp_path))
    monkeypatch.setattr(hip, "Kernel", _LoadedModule)
    calls = []
    real = hip.compile_hip

    def counting(*a, **k):
        calls.append(a[1])
        return real(*a, **k)
    monkeypatch.setattr(hip, "compile_hip", counting)
    return tmp_path, calls


def _build(block=256):
    f32p = tp.pointer_type(tp.float32)
    jf = J.JITFunction(_kernel)
    types = {"x_ptr": (f32p, "a16"), "o_ptr": (f32p, "a16"), "n": (tp.int32, "d16")}
    key = jf._key({"BLOCK": block}, types, 4, 3)
    return jf._compile(key, {"BLOCK": block}, types, 4, 3)


def _entries(path):
    return sorted(p.name.split(".", 1)[1] for p in path.iterdir())


def test_miss_writes_image_digest_and_source_then_hits(cache, monkeypatch):
    path, calls = cache
    ck = _build()
    assert len(calls) == 1
    assert _entries(path) == ["hip", "hsaco", "sha256"]
    key = J.cache_key(ck.source)
    assert (path / f"{key}.hip").read_text() == ck.source
    assert (path / f"{key}.hsaco").read_bytes() == ck.code

    def refuse(*a, **k):
        raise AssertionError("compiled although the cache holds the image")
    monkeypatch.setattr(hip, "compile_hip", refuse)
    again = _build()           # a fresh JITFunction, same kernel: served from disk
    assert again.code == ck.code and again.name == ck.name


def test_key_covers_backend_version_and_options(cache, monkeypatch):
    path, calls = cache
    ck = _build()
    k0 = J.cache_key(ck.source)
    monkeypatch.setattr(hip, "BACKEND_VERSION", hip.BACKEND_VERSION + "-next")
    assert J.cache_key(ck.source) != k0
    _build()
    assert len(calls) == 2
    monkeypatch.setattr(hip, "COMPILE_OPTIONS", hip.COMPILE_OPTIONS + ("-DNEWT_PROBE=1",))
    k2 = J.cache_key(ck.source)
    assert k2 != k0
    _build()
    assert len(calls) == 3
    assert len(list(path.glob("*.hsaco"))) == 3
    # a different specialization (constexpr) is a different source, a different entry
    assert J.cache_key(_build(block=512).source) != k2


@pytest.mark.parametrize("damage", ["flip", "truncate", "no_digest", "empty"])
def test_damaged_entry_is_rebuilt(cache, damage):
    path, calls = cache
    ck = _build()
    key = J.cache_key(ck.source)
    image = path / f"{key}.hsaco"
    data = bytearray(image.read_bytes())
    if damage == "flip":
        data[len(data) // 2] ^= 0x40
        image.write_bytes(bytes(data))
    elif damage == "truncate":
        image.write_bytes(bytes(data[:len(data) // 3]))
    elif damage == "empty":
        image.write_bytes(b"")
    else:
        os.unlink(path / f"{key}.sha256")
    again = _build()
    assert len(calls) == 2, "the damaged image was used instead of rebuilt"
    assert again.code == ck.code
    assert J._cached_image(str(image)) == ck.code     # repaired on disk
