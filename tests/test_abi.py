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


def test_config_check_refuses_head_dims_without_an_attention_kernel():
    """head_dim 96 passes the reference's own check (a multiple of 16,
    src/config.rs:70) but has no device attention instance: the library
    refuses it up front with FG_E_SHAPE instead of launching nothing."""
    from dataclasses import replace
    from ferrolm_amd import gpu
    from ferrolm_amd.weights import shape
    base = shape("smollm2-135m")
    gpu.check_config(base)  # head_dim 64: accepted
    for hd in (16, 32, 128):
        gpu.check_config(replace(base, head_dim=hd, heads=8, kv_heads=2))
    for hd in (48, 80, 96, 112):
        with pytest.raises(gpu.FgError, match=f"head_dim {hd}"):
            gpu.check_config(replace(base, head_dim=hd, heads=6, kv_heads=2))
    with pytest.raises(gpu.FgError, match="unsupported model shape"):
        gpu.check_config(replace(base, heads=9, kv_heads=2))  # src/config.rs:70: heads % kv_heads


def test_model_arrays_are_checked_before_upload():
    """A host model whose arrays are short or of the wrong type raises
    ValueError in the binding, before any pointer reaches the library."""
    import numpy as np
    from dataclasses import replace
    from ferrolm_amd import gpu
    from ferrolm_amd.weights import INT4, Matrix
    good = Matrix(INT4, 64, 64, q=np.zeros(64 * 32, np.uint8), s=np.zeros(64 * 2, np.float32))
    gpu.check_matrix(good, "w")
    with pytest.raises(ValueError, match="codes"):
        gpu.check_matrix(replace(good, q=np.zeros(64 * 31, np.uint8)), "w")
    with pytest.raises(ValueError, match="scales"):
        gpu.check_matrix(replace(good, s=np.zeros(64 * 2, np.float64)), "w")
    with pytest.raises(ValueError, match="bf16"):
        gpu.check_matrix(Matrix(0, 32, 32, bf16=np.zeros(32 * 32, np.float32)), "w")
