"""The C-ABI library loads on the CPU and exports every symbol include/snnk.h declares."""
import ctypes
import pathlib
import re

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "snnk.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(snnk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "snnk_lif_forward" in syms and "snnk_version" in syms


def test_library_exports_all_declared_symbols():
    from snnk import _abi
    lib = _abi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), f"libsnnk.so does not export {name}"
    for name in _abi.PROTOTYPES:
        assert name in declared_symbols(), f"{name} bound in _abi but not declared in snnk.h"
    assert lib.snnk_version() >= 100
    assert lib.snnk_status_string(-1) == b"invalid argument"


def test_invalid_arguments_rejected_without_gpu():
    """Argument validation happens before any HIP call."""
    from snnk import _abi
    lib = _abi.lib()
    # negative T
    st = lib.snnk_lif_forward(None, 0, None, None, None, 0, 1.0, None, None, None, 0,
                              None, -1, 10, 1, 1, 0, 0.5, 0.5, 0.0, 0, None)
    assert st == _abi.EINVAL
    # empty problem is a no-op success
    st = lib.snnk_lif_forward(None, 0, None, None, None, 0, 1.0, None, None, None, 0,
                              None, 0, 10, 1, 1, 0, 0.5, 0.5, 0.0, 0, None)
    assert st == _abi.OK
    # bad threshold mode
    st = lib.snnk_lif_forward(ctypes.c_void_p(16), 0, None, None, None, 7, 1.0, None, None,
                              ctypes.c_void_p(16), 0, None, 4, 10, 1, 1, 0, 0.5, 0.5, 0.0,
                              0, None)
    assert st == _abi.EINVAL


def test_workspace_size_queries_without_gpu():
    """The split-K workspace size is pure host arithmetic: no split (1) needs
    none, a deep small-M layer gets a split and a ticket array + partials."""
    from snnk import _abi
    for name in _abi.SIZE_PROTOTYPES:
        assert name in declared_symbols(), name
    size = lambda *a: _abi.lib().snnk_conv3x3_bn_lif_ws_size(*a)  # noqa: E731
    # T, B, H, W, Cin, Cout, pool, preact, tile_hint, splits
    assert size(4, 32, 4, 4, 512, 512, 0, 0, -1, 1) == 0
    n = size(4, 32, 4, 4, 512, 512, 0, 0, 2, 4)          # 128x128 tiles, 4 splits
    tiles = (2048 // 128) * (512 // 128)
    assert n == 65536 * 4 + tiles * 4 * 128 * 128 * 4    # fixed ticket region + partials
    assert size(4, 32, 4, 4, 512, 512, 0, 0, -1, 0) > 0  # auto split for a deep layer
    assert size(4, 32, 4, 4, 500, 512, 0, 0, -1, 0) == _abi.EUNSUPPORTED
    assert size(4, 32, 4, 4, 512, 512, 1, 1, -1, 0) == _abi.EINVAL   # preact + pool
    lin = _abi.lib().snnk_linear_bias_lif_ws_size
    assert lin(4, 32, 4096, 4096, 0, -1, 1) == 0 and lin(4, 32, 4096, 4096, 0, -1, 0) > 0
    assert _abi.lib().snnk_status_string(_abi.EWORKSPACE) == b"workspace missing or too small"


def test_workspace_pool_keys_by_device_and_stream():
    """Split-K calls on two streams must not share a workspace: the pool hands
    each (device, stream) its own buffer, grows one without touching the
    others, and refuses to grow during graph capture."""
    import pytest
    import torch
    from snnk._workspace import WorkspacePool

    made = []

    def alloc(dev, nbytes):
        made.append((dev, nbytes))
        return torch.zeros(nbytes, dtype=torch.uint8)

    pool = WorkspacePool(alloc=alloc, min_bytes=1 << 20)
    a = pool.get(0, 0x1000, 100)
    b = pool.get(0, 0x2000, 100)
    c = pool.get(1, 0x1000, 100)
    assert a is not b and a is not c and b is not c
    assert pool.get(0, 0x1000, 5000) is a                 # fits: reused
    assert pool.get(0, 0x1000, 0) is None
    big = pool.get(0, 0x1000, 3 << 20)                    # grows this stream only
    assert big is not a and big.numel() == 3 << 20
    assert pool.get(0, 0x2000, 100) is b
    assert len(made) == 4
    with pytest.raises(RuntimeError, match="capture"):
        pool.get(0, 0x3000, 100, capturing=True)          # new stream inside a capture
    assert pool.get(0, 0x2000, 100, capturing=True) is b  # existing buffer is fine


def test_noalloc_entry_point_rejects_oversized_plans_without_gpu():
    """snnk_conv3x3_bn_lif_noalloc refuses a plan whose split-K partials exceed
    its fixed 32 MiB region before any HIP call (fake, aligned pointers)."""
    from snnk import _abi
    lib = _abi.lib()
    shape = (4, 32, 16, 16, 512, 512)
    assert lib.snnk_conv3x3_bn_lif_ws_size(*shape, 0, 0, 2, 8) > (32 << 20)
    fake = ctypes.c_void_p(1 << 20)
    st = lib.snnk_conv3x3_bn_lif_noalloc(fake, fake, None, fake, None, *shape, 0,
                                         0.5, 0.5, 1.0, 0.0, 0, 2, 8, None)
    assert st == _abi.ESCRATCH
    assert b"no-alloc" in lib.snnk_status_string(st)
    # argument validation comes first, as in every entry point
    st = lib.snnk_conv3x3_bn_lif_noalloc(fake, fake, None, fake, None, 4, 32, 16, 16, 500, 512,
                                         0, 0.5, 0.5, 1.0, 0.0, 0, -1, 0, None)
    assert st == _abi.EUNSUPPORTED
