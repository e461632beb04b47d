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


def test_resumable_entry_points_validate_without_engine():
    lib = flowedge_amd.lib()
    out = (ctypes.c_float * 4)()
    rem = ctypes.c_size_t(77)
    assert lib.fe_engine_flow_begin(None, None, None, 10, 0) == 1
    assert flowedge_amd.last_error() == "Invalid arguments to fe_engine_flow_begin"
    assert lib.fe_engine_flow_advance(None, 1, out, ctypes.byref(rem)) == 1
    assert flowedge_amd.last_error() == "Invalid arguments to fe_engine_flow_advance"
    assert rem.value == 77  # not written on argument errors (engine.cc:689-692)
    assert lib.fe_engine_diffusion_begin(None, None, None, 10, 0, 0) == 1
    assert lib.fe_engine_diffusion_begin_generation(None, None, None, 10, 0, 0, 1) == 1
    assert lib.fe_engine_diffusion_advance(None, 1, out, None) == 1
    md = flowedge_amd.ConditionMetadata()
    assert lib.fe_engine_make_condition_metadata(None, 0, 0, 0, 10, 0, ctypes.byref(md)) == 1
    assert lib.fe_engine_flow_begin_request(None, None, None, ctypes.byref(md)) == 1
    assert flowedge_amd.last_error() == "Invalid versioned flow request metadata"
    amd = flowedge_amd.ActionMetadata()
    assert lib.fe_engine_flow_action_metadata(None, ctypes.byref(amd)) == 1
    lib.fe_engine_cancel_before(None, 5)  # no-op on a null engine
    # protocol/contracts.h:139-142 layouts.
    assert ctypes.sizeof(md) == 88 and ctypes.sizeof(amd) == 80
    assert ctypes.sizeof(flowedge_amd.ModelMetadata) == 96


def test_weights_digest_matches_reference_fingerprint(tmp_path):
    from oracle import fingerprint
    path = ck.write_synthetic(str(tmp_path / "tiny.safetensors"), ck.SPECS["tiny"])
    digest = flowedge_amd.weights_digest(path)
    assert digest == fingerprint.fingerprint(path)
    assert digest == flowedge_amd.weights_digest(path)  # deterministic


def _write_raw_safetensors(path, entries, metadata=True):
    """entries: (name, dtype, shape, raw bytes); writes them in the given order."""
    import json
    import struct
    header, blobs, off = {}, [], 0
    if metadata:
        header["__metadata__"] = {"format": "pt"}
    for name, dtype, shape, raw in entries:
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    js = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)) + js + b"".join(blobs))
    return str(path)


def test_fingerprint_covers_every_hash_branch_and_skips_other_dtypes(tmp_path):
    # Names of 1..40 bytes and one over 127 (cut as the reference cuts it), contents of 2..70
    # bytes (XXH64's short path, its 32-byte stripes and every tail), an I8 tensor and the
    # __metadata__ entry that the loader skips.
    from oracle import fingerprint
    import numpy as np
    rng = np.random.default_rng(3)
    entries = []
    for i in range(1, 36):
        name = ("t%02d" % i + "x" * 40)[:i + 5] if i % 3 else "n" * i
        entries.append((name, "BF16", [i], rng.integers(0, 2**16, i, dtype=np.uint16).tobytes()))
    for i in range(1, 12):
        entries.append((f"f{i}", "F32", [1, i], rng.standard_normal(i).astype(np.float32).tobytes()))
    entries.append(("q" * 140, "F32", [2, 2, 2, 2], np.arange(16, dtype=np.float32).tobytes()))
    entries.append(("skipped.int8", "I8", [3], b"\x01\x02\x03"))
    p = _write_raw_safetensors(tmp_path / "branches.safetensors", entries)
    assert flowedge_amd.weights_digest(p) == fingerprint.fingerprint(p)
    without = _write_raw_safetensors(tmp_path / "no_int8.safetensors", entries[:-1],
                                     metadata=False)
    assert flowedge_amd.weights_digest(without) == flowedge_amd.weights_digest(p)


def test_header_reader_honours_json_strings(tmp_path):
    # Tensor names and other strings holding braces, quotes, backslashes, a dtype's text or
    # escaped unicode are decoded as JSON: every F32/BF16 tensor is found under its exact name
    # (the digest hashes each name) and an I8 entry carrying the text "F32" is still skipped.
    import json
    import struct

    import numpy as np

    from oracle import fingerprint
    raw = np.arange(8, dtype=np.float32).tobytes()
    entries = [
        ("a{b}c", {"dtype": "F32", "shape": [2, 4]}),
        ('quote"d', {"dtype": "F32", "shape": [8]}),
        ("back\\slash", {"dtype": "BF16", "shape": [4, 4]}),
        ('"F32"', {"dtype": "F32", "shape": [1, 8], "note": "} { \" ]"}),
        ("caf\u00e9", {"dtype": "F32", "shape": [8]}),
        ("skip", {"dtype": "I8", "shape": [32], "comment": "\"F32\""}),
    ]
    header = {"__metadata__": {"format": "pt", "odd": "a } b { c \" d"}}
    off = 0
    for name, ent in entries:
        header[name] = dict(ent, data_offsets=[off, off + len(raw)])
        off += len(raw)
    js = json.dumps(header).encode()  # ensure_ascii: the unicode name is written as \u00e9
    assert b"\\u00e9" in js
    js += b" " * ((8 - len(js) % 8) % 8)
    path = tmp_path / "names.safetensors"
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)) + js + raw * len(entries))
    lib = flowedge_amd.lib()
    w = lib.fe_weights_load(str(path).encode())
    assert w, flowedge_amd.last_error()
    try:
        assert lib.fe_weights_size_bytes(w) == 5 * len(raw)
    finally:
        lib.fe_weights_free(w)
    names = [t[0] for t in fingerprint.tensors_in_order(str(path))]
    assert names == ["a{b}c", 'quote"d', "back\\slash", '"F32"', "caf\u00e9"]
    assert flowedge_amd.weights_digest(str(path)) == fingerprint.fingerprint(str(path))


def test_header_reader_rejects_malformed_json(tmp_path):
    import struct
    good = b'{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}'
    for bad in (b'{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}',  # unclosed
                b'{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},}',  # trailing comma
                b'{"w\\x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}',  # bad escape
                b'{"w":{"dtype":"F32","shape":[1,],"data_offsets":[0,4]}}',  # bad list
                b'{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,8]}}'):  # out of bounds
        for body, ok in ((good, True), (bad, False)):
            path = tmp_path / "h.safetensors"
            with open(path, "wb") as f:
                f.write(struct.pack("<Q", len(body)) + body + b"\0\0\0\0")
            w = flowedge_amd.lib().fe_weights_load(str(path).encode())
            assert bool(w) == ok, (body, flowedge_amd.last_error())
            if w:
                flowedge_amd.lib().fe_weights_free(w)
            else:
                assert flowedge_amd.last_error() != ""


def test_fingerprint_sensitivity(tmp_path):
    # core_model_tests.cc:392-393: equal inputs give equal digests, any change another digest.
    import numpy as np
    a = np.arange(12, dtype=np.float32).tobytes()
    base = [("w", "F32", [3, 4], a), ("b", "F32", [4], a[:16])]
    variants = {
        "base": base,
        "content": [("w", "F32", [3, 4], a[:-1] + b"\x7f"), base[1]],
        "name": [("W", "F32", [3, 4], a), base[1]],
        "shape": [("w", "F32", [4, 3], a), base[1]],
        "order": [base[1], base[0]],
        "dtype": [("w", "BF16", [6, 4], a), base[1]],
    }
    digests = {k: flowedge_amd.weights_digest(_write_raw_safetensors(tmp_path / f"{k}.st", v))
               for k, v in variants.items()}
    assert len(set(digests.values())) == len(digests)
    again = flowedge_amd.weights_digest(_write_raw_safetensors(tmp_path / "again.st", base))
    assert again == digests["base"]


def test_plain_c_caller_links_and_runs(tmp_path):
    # A C99 program built against include/flowedge.h and linked with -lflowedge_amd, as a
    # reference C caller would switch (examples/core/diffusion_sample.cc:26-50).
    import shutil
    import subprocess
    from oracle import fingerprint
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    lib_dir = os.path.join(ROOT, "flowedge_amd")
    exe = str(tmp_path / "abi_consumer")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "c", "abi_consumer.c"), "-L", lib_dir,
                    "-lflowedge_amd", f"-Wl,-rpath,{lib_dir}", "-o", exe], check=True)
    path = ck.write_synthetic(str(tmp_path / "tiny.safetensors"), ck.SPECS["tiny"])
    out = subprocess.run([exe, path], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "ok " + fingerprint.fingerprint(path)
