"""The reference-side ctypes binding printed in INTEGRATION.md stays in step with
the C ABI: the block is executed against the built library (its ABI-version
guard runs) and its struct must equal the header's byte for byte, through the
ctypes mirror that tests/test_capi.py checks with offsetof (no GPU needed)."""

import ctypes
import re

import pytest

from strata_amd import _lib

from .conftest import ROOT

DOC = ROOT / "INTEGRATION.md"


def _stub_source() -> str:
    text = DOC.read_text()
    m = re.search(r"## 2\. The binding.*?```python\n(.*?)```", text, flags=re.S)
    assert m, "INTEGRATION.md section 2 has no python block"
    return m.group(1)


@pytest.fixture(scope="module")
def stub_ns():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built; run __graft_entry__.build()")
    _lib.load()  # torch first, as the stub's own import order does
    src = _stub_source()
    assert 'ctypes.CDLL("libstrata_hip.so")' in src
    src = src.replace('ctypes.CDLL("libstrata_hip.so")', f"ctypes.CDLL({str(_lib.LIB_PATH)!r})")
    ns: dict = {}
    exec(compile(src, str(DOC), "exec"), ns)
    return ns


def test_stub_checks_the_abi_version(stub_ns):
    src = _stub_source()
    assert "strata_hip_abi_version()" in src
    assert f"!= {_lib.ABI_VERSION}" in src, "the stub's version guard names another ABI version"
    assert stub_ns["lib"].strata_hip_abi_version() == _lib.ABI_VERSION


def test_stub_struct_matches_the_abi(stub_ns):
    stub = stub_ns["Na3dArgs"]
    ref = _lib.Na3dArgs
    assert ctypes.sizeof(stub) == ctypes.sizeof(ref)
    assert [f for f, _ in stub._fields_] == [f for f, _ in ref._fields_]
    for (name, t_stub), (_, t_ref) in zip(stub._fields_, ref._fields_):
        assert getattr(stub, name).offset == getattr(ref, name).offset, name
        assert ctypes.sizeof(t_stub) == ctypes.sizeof(t_ref), name


def test_stub_sets_the_lse_pointer_to_null(stub_ns):
    """A maintainer copying the stub passes lse = NULL (no statistics written)."""
    src = _stub_source()
    assert re.search(r"a\.lse\s*=\s*None", src)
    a = stub_ns["Na3dArgs"]()
    assert a.lse is None
