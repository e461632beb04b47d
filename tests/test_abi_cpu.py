"""C ABI checks that need no GPU: the library loads, exports every declared symbol, validates
arguments and fails closed without a device."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

import flowedge_amd
from flowedge_amd import checkpoint as ck

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions() -> list[str]:
    text = open(os.path.join(ROOT, "include", "flowedge.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fe_\w+)\s*\(", text)))


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


def test_library_exports_every_declared_symbol():
    lib = flowedge_amd.lib()
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/flowedge.h but not exported"
    assert set(names) == set(flowedge_amd.EXPORTS)


def test_null_and_missing_paths_fail_with_message():
    lib = flowedge_amd.lib()
    assert not lib.fe_engine_load(None)
    assert "null" in flowedge_amd.last_error().lower()
    assert not lib.fe_engine_load(b"/nonexistent/model.safetensors")
    assert flowedge_amd.last_error() != ""
    assert lib.fe_engine_load_with_threads(b"/nonexistent", 9) is None


def test_null_engine_queries_are_safe():
    lib = flowedge_amd.lib()
    assert lib.fe_engine_action_dim(None) == 0
    assert lib.fe_engine_action_horizon(None) == 0
    assert lib.fe_engine_condition_dim(None) == 0
    assert lib.fe_engine_cuda_resident(None) == 0
    assert lib.fe_engine_thread_count(None) == 0
    md = flowedge_amd.DiffusionMetadata()
    assert lib.fe_engine_diffusion_metadata(None, ctypes.byref(md)) == 1
    assert lib.fe_engine_sample_diffusion(None, None, None, 10, 0, 0, None) == 1
    assert "Invalid arguments" in flowedge_amd.last_error()
    assert lib.fe_engine_diffusion_denoise(None, None, None, 1.0, None) == 1
    lib.fe_engine_free(None)
    assert lib.fe_engine_last_device_ms(None) == -1.0


def test_weights_store_is_host_only(tmp_path):
    path = ck.write_synthetic(str(tmp_path / "tiny.safetensors"), ck.SPECS["tiny"])
    lib = flowedge_amd.lib()
    w = lib.fe_weights_load(path.encode())
    assert w
    size = lib.fe_weights_size_bytes(w)
    assert 17 * 2**20 < size < 18 * 2**20  # tiny U-Net: 17.7 MiB of F32 tensors
    lib.fe_weights_free(w)


def test_malformed_checkpoint_is_rejected(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(b"\x10\x00\x00\x00\x00\x00\x00\x00{\"a\":{\"dtype\"}")
    lib = flowedge_amd.lib()
    assert not lib.fe_weights_load(str(p).encode())
    assert flowedge_amd.last_error() != ""


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device error path")
def test_load_without_gpu_fails_closed(tmp_path):
    path = ck.write_synthetic(str(tmp_path / "tiny.safetensors"), ck.SPECS["tiny"])
    with pytest.raises(RuntimeError, match="HIP device|GPU"):
        flowedge_amd.Engine(path)


def test_invalid_threads_env_is_rejected(tmp_path, monkeypatch):
    monkeypatch.setenv("FLOWEDGE_THREADS", "99")
    lib = flowedge_amd.lib()
    assert not lib.fe_engine_load(b"/whatever")
    assert "FLOWEDGE_THREADS" in flowedge_amd.last_error()


def test_force_host_fails_closed(tmp_path, monkeypatch):
    path = ck.write_synthetic(str(tmp_path / "tiny.safetensors"), ck.SPECS["tiny"])
    monkeypatch.setenv("FLOWEDGE_CUDA_FORCE_HOST", "1")
    with pytest.raises(RuntimeError, match="no host kernels"):
        flowedge_amd.Engine(path)


def test_invalid_meta_rejected_before_device(tmp_path):
    tensors = dict(ck.synthetic_tensors(ck.SPECS["tiny"]))
    tensors["dp.meta"] = tensors["dp.meta"].copy()
    tensors["dp.meta"][7] = 4.0  # even kernel size
    p = str(tmp_path / "bad_meta.safetensors")
    ck.write_safetensors(p, tensors.items())
    with pytest.raises(RuntimeError, match="dp.meta"):
        flowedge_amd.Engine(p)
