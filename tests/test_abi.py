"""The C-ABI library loads, exports every symbol include/ovfq.h declares, and validates arguments before
any device work (no compute calls here: this runs without a GPU)."""
import ctypes

import numpy as np
import pytest

import overfit_amd
from overfit_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _lib.declared_symbols()
    assert len(declared) >= 25
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), "binding table out of date with the header"


def test_version_and_error_string():
    lib = _lib.load()
    assert lib.ovfq_version().startswith(b"ovfq")
    assert isinstance(lib.ovfq_last_error(), bytes)


def test_null_arguments_are_rejected_before_device_work():
    lib = _lib.load()
    assert lib.ovfq_ctx_create(0, None) == _lib.OVFQ_ERR_NULL
    h = ctypes.c_void_p()
    assert lib.ovfq_weight_create(None, 12, None, 0, None, 256, 1, ctypes.byref(h)) == _lib.OVFQ_ERR_NULL
    assert b"NULL" in lib.ovfq_last_error()
    assert lib.ovfq_project(None, None, None, 1, None, None) == _lib.OVFQ_ERR_NULL
    assert lib.ovfq_quantize_q8k(None, None, 1, 256, None, None, None) == _lib.OVFQ_ERR_NULL
    assert lib.ovfq_ctx_destroy(None) == _lib.OVFQ_ERR_NULL
    assert lib.ovfq_ctx_set_batched_kernel(None, 0) == _lib.OVFQ_ERR_NULL
    assert lib.ovfq_weight_destroy(None) == _lib.OVFQ_ERR_NULL


def test_python_mirror_validates_shapes_before_touching_the_device():
    blocks = np.zeros(144, np.uint8)
    with pytest.raises(overfit_amd.OverfitArgumentOutOfRangeError):
        overfit_amd.Q4KWeight(blocks, 0, 1)
    with pytest.raises(overfit_amd.OverfitArgumentError):
        overfit_amd.Q4KWeight(blocks, 100, 1)  # inputSize % 256 != 0
    with pytest.raises(overfit_amd.OverfitArgumentError):
        overfit_amd.Q4KWeight(blocks, 512, 1)  # region smaller than 2 blocks
    with pytest.raises(overfit_amd.OverfitArgumentNullError):
        overfit_amd.Q4KWeight(None, 256, 1)
    with pytest.raises(overfit_amd.OverfitArgumentError):
        overfit_amd.Q8Weight(np.zeros(64, np.int8), np.zeros(2, np.float32), 33, 1)
    with pytest.raises(overfit_amd.OverfitArgumentError):
        overfit_amd.Q4KDotKernel.QuantizeActivationQ8K(np.zeros(300, np.float32), np.zeros(300, np.int8),
                                                      np.zeros(2, np.float32), np.zeros(32, np.int16))
    with pytest.raises(overfit_amd.OverfitArgumentError):
        overfit_amd.Q4KDotKernel.QuantizeActivationQ8K(np.zeros(256, np.float32), np.zeros(255, np.int8),
                                                      np.zeros(1, np.float32), np.zeros(16, np.int16))
    with pytest.raises(overfit_amd.OverfitArgumentError):
        overfit_amd.Q8DotKernel.Quantize(np.zeros(33, np.float32), np.zeros(33, np.int8), np.zeros(2, np.float32))


def test_product_package_does_not_import_the_oracle():
    import os
    import re

    pkg = os.path.dirname(overfit_amd.__file__)
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"\boracle\b|ovfq_oracle|cpu_baseline", text), f


def test_kernels_never_bit_cast_a_vector_element():
    # __builtin_bit_cast(T, v.y) on an ext_vector element reads element 0 with this hipcc (it narrowed the Q8_K
    # quantiser's 16-byte load to one dword); kernels copy lanes to scalars first (as_float).
    import os
    import re

    csrc = os.path.join(os.path.dirname(overfit_amd.__file__), "csrc")
    pat = re.compile(r"__builtin_bit_cast\s*\([^,]+,\s*[\w\.\[\]]+\.[xyzw]\s*\)")
    for f in os.listdir(csrc):
        text = open(os.path.join(csrc, f)).read()
        assert not pat.search(text), f


def test_multi_read_lds_asm_outputs_are_early_clobber():
    # An inline-asm block that issues several LDS reads before one wait must mark every output early-clobber ("=&v"):
    # a read's data can land while a later read of the block still needs its address register, and without the
    # marker the compiler may give both the same VGPR. (The MoE combine's token/weight read once got its weight
    # address overwritten by the token this way, giving wrong combine weights depending on timing.)
    import os
    import re

    csrc = os.path.join(os.path.dirname(overfit_amd.__file__), "csrc")
    for name in sorted(os.listdir(csrc)):
        if not name.endswith((".hip", ".h", ".cpp")):
            continue
        text = open(os.path.join(csrc, name)).read()
        for m in re.finditer(r"asm\s+volatile\s*\((.*?)\);", text, re.S):
            body = m.group(1)
            template, _, operands = body.partition(":")
            if template.count("ds_read") < 2:
                continue
            outputs = operands.split(":")[0]
            plain = re.findall(r'"=v"', outputs)
            assert not plain, f"{name}: multi-read asm block with non-early-clobber outputs: {template[:60]!r}"
