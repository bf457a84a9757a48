"""CPU checks of the native boundary: exports, prototypes, RTC sources (no GPU calls)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pacho_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(hp_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_documented_entry_points():
    names = _declared()
    for required in ("hp_init", "hp_gemm", "hp_gemv", "hp_dot", "hp_norm", "hp_reduce", "hp_philox", "hp_rtc_compile"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from openpacho import _hip_lib

    lib = _hip_lib.load()
    missing = [name for name in _declared() if not hasattr(lib, name)]
    assert not missing, missing
    assert set(_declared()) == set(_hip_lib.PROTOTYPES)
    assert lib.hp_version().decode().startswith("pacho_hip")
    assert lib.hp_last_error() is not None


def test_library_has_gfx950_code_objects():
    from openpacho import _hip_lib

    blob = _hip_lib.library_path().read_bytes()
    assert b"gfx950" in blob


def test_status_codes_map_to_reference_exception_types():
    from openpacho import _hip_lib

    class FakeLib:
        def hp_last_error(self):
            return b"detail"

    with pytest.raises(ValueError, match="detail"):
        _hip_lib.check(FakeLib(), _hip_lib.HP_E_INVALID, "op")
    with pytest.raises(NotImplementedError):
        _hip_lib.check(FakeLib(), _hip_lib.HP_E_UNSUPPORTED, "op")
    for code in (_hip_lib.HP_E_HIP, _hip_lib.HP_E_OOM, _hip_lib.HP_E_RTC, _hip_lib.HP_E_INJECTED):
        with pytest.raises(RuntimeError):
            _hip_lib.check(FakeLib(), code, "op")
    _hip_lib.check(FakeLib(), _hip_lib.HP_OK, "op")


# ---- hipRTC sources of the lowering compile for gfx950 (offline, no device) --------------

_RTC = None


def _rtc():
    global _RTC
    if _RTC is None:
        for candidate in ("/opt/rocm/lib/libhiprtc.so", "libhiprtc.so"):
            try:
                _RTC = ctypes.CDLL(candidate)
                break
            except OSError:
                continue
        else:
            pytest.skip("libhiprtc not available")
    return _RTC


def _compiles(source):
    rtc = _rtc()
    program = ctypes.c_void_p()
    assert rtc.hiprtcCreateProgram(ctypes.byref(program), source.encode(), b"t.hip", 0, None, None) == 0
    options = [b"--offload-arch=gfx950", b"-O3", b"-ffp-contract=off", b"-Xclang", b"-target-feature", b"-Xclang", b"-packed-fp32-ops"]
    status = rtc.hiprtcCompileProgram(program, len(options), (ctypes.c_char_p * len(options))(*options))
    size = ctypes.c_size_t()
    rtc.hiprtcGetProgramLogSize(program, ctypes.byref(size))
    log = ctypes.create_string_buffer(size.value + 1)
    rtc.hiprtcGetProgramLog(program, log)
    rtc.hiprtcDestroyProgram(ctypes.byref(program))
    return status, log.value.decode(errors="replace")


class _Operand:
    def __init__(self, shape, dtype, scalar=False):
        self.shape, self.dtype, self._host_scalar = tuple(shape), np.dtype(dtype), scalar


EAGER_CASES = [
    ("add", [_Operand((8, 4), "f4"), _Operand((4,), "f4")], (8, 4), "f4"),
    ("divide", [_Operand((8,), "f8"), _Operand((), "f8", True)], (8,), "f8"),
    ("tanh", [_Operand((8,), "f4")], (8,), "f4"),
    ("where", [_Operand((8,), "?"), _Operand((8,), "i8"), _Operand((), "i8", True)], (8,), "i8"),
    ("cast", [_Operand((8,), "f8")], (8,), "i4"),
    ("absolute", [_Operand((8,), "i4")], (8,), "i4"),
    ("isfinite", [_Operand((8,), "f4")], (8,), "?"),
    ("power", [_Operand((8,), "f8"), _Operand((), "f8", True)], (8,), "f8"),
    ("multiply", [_Operand((8,), "?"), _Operand((8,), "?")], (8,), "?"),
    ("negative", [_Operand((8,), "u8")], (8,), "u8"),
    ("less_equal", [_Operand((8,), "u4"), _Operand((8,), "u4")], (8,), "?"),
]


@pytest.mark.parametrize("name,args,shape,dtype", EAGER_CASES, ids=[c[0] for c in EAGER_CASES])
def test_eager_sources_compile(name, args, shape, dtype):
    from openpacho._hip_lowering import eager_source

    source, grid = eager_source(name, args, shape, dtype)
    status, log = _compiles(source)
    assert status == 0, log
    assert grid >= 1


class _Node:
    def __init__(self, op, shape, dtype, inputs=(), resolved=(), attrs=None):
        self.op, self.shape, self.dtype = op, tuple(shape), np.dtype(dtype)
        self.inputs, self.resolved, self.attrs = tuple(inputs), tuple(np.dtype(r) for r in resolved), attrs or {}


@pytest.mark.parametrize("operation,dtype", [("sum", "f4"), ("min", "f4"), ("max", "f8"), ("max", "i8"), ("min", "u4"), ("min", "?")])
def test_map_reduce_sources_compile(operation, dtype):
    from openpacho._hip_lowering import HIPLowering

    x = _Node("input", (8, 100), dtype)
    attrs = {"axes": (1,), "keepdims": False}
    if operation != "sum":
        attrs["operation"] = operation
    node = _Node("reduce", (8,), dtype, (x,), attrs=attrs)
    _, (source, count, chunks) = HIPLowering(None).prepare_map_reduce(node, (), [x])
    status, log = _compiles(source)
    assert status == 0, log
    assert (count, chunks) == (8, 1)


def test_fused_mlp_epilogue_source_compiles_and_keeps_per_node_rounding():
    from openpacho._hip_lowering import HIPLowering

    f4 = np.dtype("f4")
    h = _Node("input", (8, 1024), f4)
    b = _Node("input", (1024,), f4)
    add = _Node("add", (8, 1024), f4, (h, b), (f4, f4, f4))
    th = _Node("tanh", (8, 1024), f4, (add,), (f4, f4))
    red = _Node("reduce", (8,), f4, (th,), attrs={"axes": (1,), "keepdims": False})
    _, (source, count, chunks) = HIPLowering(None).prepare_map_reduce(red, [add, th], [h, b])
    assert "tanh" in source and "% 1024LL" in source
    status, log = _compiles(source)
    assert status == 0, log


def test_host_small_blocks_match_the_pool_smallest_size_class():
    # The backend hands any waiting small block to any request of at most
    # _SMALL_BLOCK bytes, which is sound only while every such request gets a
    # block of the pool's smallest size class (runtime.hip size_class).
    from openpacho import _hip

    source = (ROOT / "open-pacho_amd" / "csrc" / "runtime.hip").read_text()
    match = re.search(r"if \(bytes <= (\d+)\) return (\d+);", source)
    assert match, "size_class's smallest class not found"
    assert int(match.group(1)) == int(match.group(2)) == _hip._SMALL_BLOCK
