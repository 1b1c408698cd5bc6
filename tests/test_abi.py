"""CPU checks of the C-ABI library: it loads, exports every symbol include/ha.h declares, and its host-side
validation returns the documented status codes before touching a device (no compute without a GPU)."""
import ctypes
import os
import re

import pytest

import hybrid_attention as ha

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "ha.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ha_[a-z_0-9]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = ha.load_library()
    names = _declared()
    assert "ha_forward" in names and len(names) >= 17
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version_matches_header():
    src = open(os.path.join(ROOT, "include", "ha.h")).read()
    v = int(re.search(r"#define HA_ABI_VERSION (\d+)", src).group(1))
    assert ha.load_library().ha_abi_version() == v


def _cfg(**over):
    c = ha.model_config(["linear_attention", "full_attention"])
    c.update(over)
    return c


@pytest.mark.parametrize("over,msg", [
    (dict(kinds=[0, 7]), "unknown layer kind"),
    (dict(batch=0), "batch"),
    (dict(DK=64), "d_k = d_v = 128"),
    (dict(conv_k=3), "conv kernel 4"),
    (dict(lin_stride=8000), "lin_stride"),
    (dict(lin_stride=8260), "multiple of 8"),
    (dict(HQ=6), "4 query heads per KV head"),
    (dict(HD=128), "head_dim 256"),
    (dict(rot_dim=48), "rotary_dim"),
    (dict(full_stride=4096), "full_stride"),
    (dict(eps=1e-5), "eps"),
    (dict(lin_dtype=5), "lin_dtype"),
])
def test_create_rejects_bad_configs_before_touching_a_device(over, msg):
    with pytest.raises(ha.HAError) as ei:
        ha.Engine(_cfg(**over))
    assert ei.value.code == ha.HA_ERR_ARG and msg in str(ei.value)


def test_null_handles_are_rejected():
    lib = ha.load_library()
    assert lib.ha_destroy(None) == ha.HA_ERR_HANDLE
    assert lib.ha_forward(None, 1, None, None, None, None, None) == ha.HA_ERR_HANDLE
    p = ctypes.c_int()
    assert lib.ha_snapshot_tokens(None, ctypes.byref(p)) == ha.HA_ERR_HANDLE
    assert lib.ha_snapshot_release(None) == ha.HA_ERR_HANDLE
    assert lib.ha_synchronize(None) == ha.HA_ERR_HANDLE
    assert b"invalid" in lib.ha_last_error()


def test_no_device_is_a_device_error_not_a_fallback():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(ha.HAError) as ei:
        ha.Engine(_cfg())
    assert ei.value.code == ha.HA_ERR_DEVICE


def test_forged_handles_are_refused_not_read():
    """Handles are looked up in the library's registries before any field is read: a block of memory that merely
    starts with a handle's magic value (as a freed handle would) is refused with HA_ERR_HANDLE."""
    lib = ha.load_library()
    buf = (ctypes.c_uint32 * 64)()
    p = ctypes.c_int()
    for magic in (0x48415350, 0x48414D4E, 0x4841454E):  # snapshot, MatMulNBits, engine
        buf[0] = magic
        h = ctypes.cast(buf, ctypes.c_void_p)
        assert lib.ha_snapshot_tokens(h, ctypes.byref(p)) == ha.HA_ERR_HANDLE
        assert lib.ha_snapshot_layout(h, ctypes.byref(p), ctypes.byref(p)) == ha.HA_ERR_HANDLE
        assert lib.ha_snapshot_read(h, 0, b"state", ctypes.cast(buf, ctypes.c_void_p), 4) == ha.HA_ERR_HANDLE
        assert lib.ha_snapshot_release(h) == ha.HA_ERR_HANDLE
        assert lib.ha_snapshot_destroy(h) == ha.HA_ERR_HANDLE
        assert lib.ha_mnb_forward(h, 1, h, h, None) == ha.HA_ERR_HANDLE
        assert lib.ha_mnb_forward_noalloc(h, 1, h, h, None) == ha.HA_ERR_HANDLE
        assert lib.ha_mnb_destroy(h) == ha.HA_ERR_HANDLE
        assert lib.ha_embed(h, 1, h, h, None) == ha.HA_ERR_HANDLE
        assert lib.ha_destroy(h) == ha.HA_ERR_HANDLE
        assert lib.ha_set_stream(h, None) == ha.HA_ERR_HANDLE
        assert lib.ha_share_scratch(h, h) == ha.HA_ERR_HANDLE
        ms = ctypes.c_float()
        assert lib.ha_timer_mark(h, 0, None) == ha.HA_ERR_HANDLE
        assert lib.ha_timer_elapsed(h, 0, 0, ctypes.byref(ms)) == ha.HA_ERR_HANDLE
        assert lib.ha_timer_destroy(h) == ha.HA_ERR_HANDLE
    assert buf[0] == 0x4841454E  # nothing wrote through the forged handles
