"""The C-ABI library: it loads, exports every entry point the public headers
declare, and fails loudly (an error code, no crash, no CPU fallback) where
no GPU is present. CPU only; no compute calls."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared(header: Path):
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(f[gh]_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from ferrolm_amd import gpu
    lib = ctypes.CDLL(str(gpu.LIB_PATH))
    names = declared(ROOT / "include" / "ferro_gpu.h") + declared(ROOT / "include" / "ferro_host.h")
    assert len(names) > 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    from ferrolm_amd import gpu
    names = declared(ROOT / "include" / "ferro_gpu.h")
    assert set(names) <= set(gpu.EXPORTS), set(names) - set(gpu.EXPORTS)


def test_no_gpu_means_an_error_not_a_fallback():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from ferrolm_amd import gpu
    with pytest.raises(gpu.FgError):
        gpu.Context(0)


def test_product_code_never_imports_the_oracle():
    for p in (ROOT / "ferrolm_amd").rglob("*"):
        if p.suffix in (".py", ".hip", ".cpp", ".h"):
            t = p.read_text()
            assert "import oracle" not in t and "from oracle" not in t and "ferro_oracle" not in t, p


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 exits with status 2 and says
    why, before touching the device."""
    import subprocess
    import sys
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], cwd=root, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and not r.stdout.strip()
