"""The product path has no CPU fallback: without the HIP library every entry
point raises, and nothing in the package reaches the test oracle."""
import ast
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "welder_typical_chain_amd"


def test_missing_library_raises(monkeypatch, tmp_path):
    from welder_typical_chain_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libwtc_hip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()
    with pytest.raises(RuntimeError, match="not built"):
        _lib.check(_lib.WTC_ERR_ARG)  # reading the error message needs the library too


def _imports(path: Path):
    tree = ast.parse(path.read_text(), filename=str(path))
    for node in ast.walk(tree):
        if isinstance(node, ast.Import):
            for a in node.names:
                yield a.name
        elif isinstance(node, ast.ImportFrom):
            yield node.module or ""


def test_package_never_imports_the_oracle():
    files = sorted(PKG.rglob("*.py"))
    assert files
    for f in files:
        for mod in _imports(f):
            assert not mod.split(".")[0] == "oracle", f"{f.relative_to(ROOT)} imports {mod}"
        assert "oracle/" not in f.read_text(), f"{f.relative_to(ROOT)} names a path under oracle/"


def test_native_sources_never_include_the_oracle():
    for f in sorted((PKG / "csrc").iterdir()):
        if f.suffix in (".hip", ".cpp", ".h"):
            text = f.read_text()
            assert "wtc_oracle" not in text and '#include "oracle' not in text, f.name
