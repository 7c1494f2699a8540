"""CPU checks of the C ABI: the library loads (no GPU needed to dlopen) and
exports every entry point include/gs_sampler.h declares."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    h = open(os.path.join(ROOT, "include", "gs_sampler.h")).read()
    h = re.sub(r"/\*.*?\*/", "", h, flags=re.S)
    return sorted(set(re.findall(r"\b(gs_[a-z_]+)\s*\(", h)))


def test_header_declares_api():
    names = declared()
    for n in ("gs_sampler_create", "gs_sample", "gs_sample_batch", "gs_sampler_set_seed"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import gs_sampler
    lib = gs_sampler.load_library()
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(gs_sampler.EXPORTS) == declared()


def test_limits_and_version():
    import gs_sampler
    lib = gs_sampler.load_library()
    v, w = ctypes.c_uint32(), ctypes.c_uint32()
    assert lib.gs_limits(ctypes.byref(v), ctypes.byref(w)) == 0
    assert v.value == 1 << 22 and w.value >= 1024
    assert b"gfx950" in lib.gs_version()


def test_null_arguments_rejected_without_gpu():
    import gs_sampler
    lib = gs_sampler.load_library()
    assert lib.gs_sampler_create(None, 0, None) == gs_sampler.GS_ERR_INVALID
    assert lib.gs_sampler_destroy(None) == gs_sampler.GS_ERR_INVALID
    assert lib.gs_sample(None, None, 0, None, 0, None) == gs_sampler.GS_ERR_INVALID
    assert lib.gs_sample_batch(None, None, 1, 1, 1, None, None, 0, None, 0, None, None, None,
                               None) == gs_sampler.GS_ERR_INVALID


def test_workload_shapes():
    import workloads
    w = workloads.make("c2", B=2)
    assert w["logits"].shape == (2, 128256) and w["recent"].shape == (2, 128)
    assert workloads.algorithmic_bytes_per_row(152064, 0) == 608264
    w = workloads.make("c4", B=8)
    assert set(w["params"]["top_k"]) <= {0, 1, 20, 100}
    d, _ = workloads.lcg_stream(42, 2)
    assert float(d[0]) == 0.0
