"""The C ABI library (no GPU needed): it loads, exports every function that
include/adasplash.h declares, and validates arguments on the host."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "adasplash.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*\*?\s*(asa_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from splash_attention import _lib

    return _lib.load()


def test_header_declares_what_the_binding_binds():
    from splash_attention import _lib

    assert _declared() == sorted(_lib.EXPORTS)


def _header_fields(struct):
    """Field names of `typedef struct <struct> { ... }` in the C header, in order."""
    text = open(os.path.join(ROOT, "include", "adasplash.h")).read()
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        # "type a, b, c" / "type *a" / "type a[3]"
        m = re.match(r"^(?:const\s+)?\w+\s*\**\s*(.*)$", decl, re.S)
        for part in m.group(1).split(","):
            names.append(re.sub(r"[\s*]|\[.*\]", "", part))
    return names


def _integration_fields(cls):
    """Field names of the ctypes class `cls` in the integration guide's
    binding example (the guide at the repository root)."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = re.search(r"class %s\(ctypes\.Structure\):\s*_fields_ = (.*?\])\n\n" % cls, text, re.S)
    return re.findall(r'"(\w+)"', block.group(1))


def test_struct_layouts_agree_header_binding_and_docs():
    """asa_problem, asa_state and asa_sizes: the header, the package's ctypes
    binding and the integration guide's example list the same fields in the same
    order (a caller whose struct lacks a trailing field, such as the state's
    status word, hands the library memory past its struct)."""
    from splash_attention import _lib

    for struct, cls in (("asa_problem", _lib.Problem), ("asa_state", _lib.State),
                        ("asa_sizes", _lib.Sizes)):
        want = _header_fields(struct)
        assert [f[0] for f in cls._fields_] == want, struct
        assert _integration_fields(cls.__name__) == want, struct


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    from splash_attention import _lib

    assert lib.asa_abi_version() == _lib.ABI_VERSION
    hdr = open(os.path.join(ROOT, "include", "adasplash.h")).read()
    assert f"#define ASA_ABI_VERSION {_lib.ABI_VERSION}" in hdr


def _problem(**kw):
    from splash_attention import _lib

    base = dict(batch=4, heads=16, nq=4096, nk=4096, head_dim=64, k_keep=32, block_m=64,
                block_n=64, alpha=1.5, sm_scale=0.125, dtype=_lib.DTYPE_BF16)
    base.update(kw)
    return _lib.Problem(**base)


def test_query_sizes_headline():
    from splash_attention import _lib

    z = _lib.query_sizes(_problem())
    rows = 64 * 4096
    assert z.taus == rows * 4 and z.norms == rows * 4
    assert z.mask == 64 * 64 * 64
    assert z.q_ptr == 64 * 65 * 4 and z.k_ptr == 64 * 65 * 4
    assert z.q_list == 64 * 64 * 64 * 4 and z.k_list == z.q_list
    assert z.topk_idx == rows * 32 * 4
    assert z.workspace >= 2 * rows * 4


@pytest.mark.parametrize("bad,code,msg", [
    (dict(head_dim=256), 1, "Head dimension too large"),
    (dict(head_dim=0), 1, "head_dim 0 must be >= 1"),
    (dict(head_dim=50), 2, "head_dim 50 must be a multiple of 8"),
    (dict(head_dim=6, dtype=0), 2, "head_dim 6 must be a multiple of 4"),
    (dict(q_strides=(-64, 64, 64)), 1, "q_strides[0] = -64"),
    (dict(k_strides=(0, 0, 68)), 1, "k_strides[2] = 68"),
    (dict(v_strides=(0, 4, 1 << 20)), 1, "v_strides[1] = 4"),
    (dict(dout_strides=(0, 0, 1 << 20)), 2, "dout row stride"),
    (dict(k_keep=0), 1, "k_keep"),
    (dict(k_keep=129), 1, "k_keep"),
    (dict(block_m=16), 2, "block_m"),
    (dict(nq=0), 1, "nq"),
    (dict(batch=0), 1, "batch"),
    (dict(dtype=7), 1, "dtype"),
    (dict(alpha=float("nan")), 1, "alpha"),
    (dict(sm_scale=float("inf")), 1, "sm_scale"),
    (dict(tau_mode=5), 1, "tau_mode"),
])
def test_invalid_problems_are_rejected_on_the_host(lib, bad, code, msg):
    from splash_attention import _lib

    p = _problem(**bad)
    z = _lib.Sizes()
    assert lib.asa_query_sizes(ctypes.byref(p), ctypes.byref(z)) == code
    assert msg in lib.asa_last_error().decode()
    # the entry points validate before touching the device
    st = _lib.State()
    rc = lib.asa_forward(ctypes.byref(p), None, None, None, None, None, None, ctypes.byref(st),
                         None, None)
    assert rc == code


def test_null_pointers_are_rejected(lib):
    from splash_attention import _lib

    p = _problem()
    st = _lib.State()
    assert lib.asa_forward(ctypes.byref(p), None, None, None, None, None, None,
                           ctypes.byref(st), None, None) == _lib.ASA_ERR_INVALID_ARGUMENT
    assert "NULL" in lib.asa_last_error().decode()
    assert lib.asa_backward(ctypes.byref(p), 5, None, None, None, None, None, None, None,
                            ctypes.byref(st), None, None, None, None, None) == \
        _lib.ASA_ERR_INVALID_ARGUMENT
    assert "grad_mode" in lib.asa_last_error().decode()


def test_any_whole_chunk_head_dim_and_strides_are_accepted(lib):
    """head_dim: any multiple of 8 (16-bit) or 4 (fp32) up to 128; strides:
    whole chunks, e.g. a [B, N, H, d] tensor viewed as [B, H, N, d] and K
    shared across heads (head stride 0)."""
    from splash_attention import _lib

    z = _lib.Sizes()
    for d, dt in ((8, _lib.DTYPE_BF16), (40, _lib.DTYPE_F16), (96, _lib.DTYPE_BF16),
                  (4, _lib.DTYPE_F32), (100, _lib.DTYPE_F32), (128, _lib.DTYPE_F32)):
        assert lib.asa_query_sizes(ctypes.byref(_problem(head_dim=d, dtype=dt)),
                                   ctypes.byref(z)) == 0, lib.asa_last_error()
    B, H, N, d = 4, 16, 4096, 64
    p = _problem(q_strides=(N * H * d, d, H * d), k_strides=(N * d, 0, d),
                 v_strides=(0, 0, 0), dout_strides=(N * H * d, d, H * d))
    assert lib.asa_query_sizes(ctypes.byref(p), ctypes.byref(z)) == 0, lib.asa_last_error()


def test_misaligned_tensors_are_rejected(lib):
    from splash_attention import _lib

    p = _problem()
    st = _lib.State()
    a, bad = 1 << 20, (1 << 20) + 8   # stand-in addresses: never dereferenced
    rc = lib.asa_forward(ctypes.byref(p), bad, a, a, a, a, a, ctypes.byref(st), a, None)
    assert rc == _lib.ASA_ERR_INVALID_ARGUMENT
    assert "16-byte aligned" in lib.asa_last_error().decode()
    rc = lib.asa_backward(ctypes.byref(p), 0, a, a, a, a, a, None, a, ctypes.byref(st), a, a,
                          bad, a, None)
    assert rc == _lib.ASA_ERR_INVALID_ARGUMENT
    assert "16-byte aligned" in lib.asa_last_error().decode()


def test_error_string_is_cleared_on_success(lib):
    from splash_attention import _lib

    z = _lib.Sizes()
    bad = _problem(k_keep=0)
    lib.asa_query_sizes(ctypes.byref(bad), ctypes.byref(z))
    assert lib.asa_last_error().decode() != ""
    good = _problem()
    assert lib.asa_query_sizes(ctypes.byref(good), ctypes.byref(z)) == 0
    assert lib.asa_last_error().decode() == ""


def test_exact_tau_mode_is_forward_only(lib):
    from splash_attention import _lib

    p = _problem(tau_mode=_lib.TAU_EXACT)
    z = _lib.Sizes()
    assert lib.asa_query_sizes(ctypes.byref(p), ctypes.byref(z)) == 0
    st = _lib.State()
    rc = lib.asa_select_from_scores(ctypes.byref(p), None, None, None, ctypes.byref(st), None,
                                    None)
    assert rc == _lib.ASA_ERR_UNSUPPORTED
    assert "exact tau mode" in lib.asa_last_error().decode()
