"""CPU checks of the C ABI: the library loads (no GPU needed to dlopen) and
exports every entry point include/gs_sampler.h declares."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    import glob
    names = set()
    for path in sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))):
        h = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
        names |= set(re.findall(r"\b(gs_[a-z_]+)\s*\(", h))
    return sorted(names)


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


def test_gemv_arguments_rejected_without_gpu():
    import ctypes as C
    import gs_sampler
    lib = gs_sampler.load_library()
    h = C.c_void_p()
    blk = (C.c_uint8 * 210)()
    assert lib.gs_qmatrix_upload(14, None, 1, 256, C.byref(h)) == gs_sampler.GS_ERR_INVALID
    assert lib.gs_qmatrix_upload(14, blk, 1, 256, None) == gs_sampler.GS_ERR_INVALID
    # cols not a multiple of the block size: the reference's upload returns None
    assert lib.gs_qmatrix_upload(14, blk, 1, 128, C.byref(h)) == gs_sampler.GS_ERR_UNSUPPORTED
    assert lib.gs_qmatrix_upload(8, blk, 1, 48, C.byref(h)) == gs_sampler.GS_ERR_UNSUPPORTED
    for qt in (2, 3):                  # Q4_0, Q4_1: 32-weight blocks
        assert lib.gs_qmatrix_upload(qt, blk, 1, 48, C.byref(h)) == gs_sampler.GS_ERR_UNSUPPORTED
    assert lib.gs_qmatrix_upload(11, blk, 1, 128, C.byref(h)) == gs_sampler.GS_ERR_UNSUPPORTED  # Q3_K
    # block types the reference's upload does not take (F32, F16, Q5_0, Q5_1, Q8_1, Q2_K, Q8_K)
    for qt in (0, 1, 6, 7, 9, 10, 15):
        assert lib.gs_qmatrix_upload(qt, blk, 1, 256, C.byref(h)) == gs_sampler.GS_ERR_UNSUPPORTED
    assert lib.gs_qmatrix_upload(14, blk, 1, 256 * 65, C.byref(h)) == gs_sampler.GS_ERR_UNSUPPORTED
    assert lib.gs_qmatrix_destroy(None) == gs_sampler.GS_ERR_INVALID
    assert lib.gs_gemv(None, None, 1, None, None) == gs_sampler.GS_ERR_INVALID


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
