"""The C-ABI library loads and exports every function include/rtq.h declares (no GPU needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "rtq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(rtq_[a-z_0-9]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ["rtq_ctx_create", "rtq_weight_create", "rtq_frozen_forward", "rtq_frozen_backward_input",
                 "rtq_frozen_row", "rtq_weight_nbytes", "rtq_linear_forward", "rtq_linear_backward",
                 "rtq_frozen_forward_d", "rtq_linear_backward_d", "rtq_debug_block_isums"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    from rust_trainer_amd import _ffi

    lib = ctypes.CDLL(_ffi.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the whole header
    assert set(declared_functions()) == set(_ffi.SIGNATURES)
    assert _ffi.lib().rtq_version().decode().startswith("rtq")


def test_code_object_is_gfx950_only():
    # the embedded code object is built for gfx950 and nothing else
    hsaco = os.path.join(ROOT, "rust_trainer_amd", "_build", "rtq_kernels.hsaco")
    if not os.path.exists(hsaco):
        pytest.skip("code object not built here")
    data = open(hsaco, "rb").read()
    assert data[:4] == b"\x7fELF"
    e_flags = int.from_bytes(data[48:52], "little")
    assert e_flags & 0xFF == 0x4F  # EF_AMDGPU_MACH_AMDGCN_GFX950
    assert (e_flags & 0x300) != 0x300  # not an xnack+ code object
    lib = open(os.path.join(ROOT, "rust_trainer_amd", "librtq.so"), "rb").read()
    assert data in lib  # embedded verbatim, loaded with hipModuleLoadData


def test_python_mirror_shapes_are_checked_before_any_device_call():
    import numpy as np

    from rust_trainer_amd import frozen

    class Fake(frozen.HipFrozen):
        def __init__(self):  # no device: only the host-side checks run
            self._rows, self._cols, self.ggml_type = 4, 32, 2

    f = Fake()
    with pytest.raises(AssertionError):
        f.forward(np.zeros(31, np.float32), 1)
    with pytest.raises(AssertionError):
        f.backward_input(np.zeros(4, np.float32), 1, np.zeros(31, np.float32))
