"""The C ABI library loads and exports what include/leatmi.h declares; argument checks reject
bad calls before any launch (host logic only: no kernel runs here)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "leatmi.h"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(leat_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from leat_amd import _lib

    if not _lib.LIB_PATH.exists():
        from leat_amd import build

        build.build()
    return _lib.lib()


def test_exports_every_declared_symbol(lib):
    names = declared()
    assert len(names) >= 10
    for name in names:
        assert getattr(lib, name) is not None, name


def test_python_binding_covers_the_header():
    from leat_amd import _lib

    missing = [n for n in declared() if n not in _lib.SIGNATURES and n not in
               ("leat_last_error", "leat_abi_version", "leat_target")]  # fmt: skip
    assert not missing


def test_identity(lib):
    assert lib.leat_target() == b"gfx950"
    assert lib.leat_abi_version() >= 1


def test_rejects_bad_arguments(lib):
    from leat_amd import _lib

    one = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_lib.LeatError, match="unsupported type 99"):
        _lib.call("leat_matvec", 99, one, 4, 256, one, one, one, 1, None, one, None)
    with pytest.raises(_lib.LeatError, match="256-weight blocks"):
        _lib.call("leat_matvec", 12, one, 4, 100, one, one, one, 1, None, one, None)
    with pytest.raises(_lib.LeatError, match="whole groups of 32"):
        _lib.call("leat_quantize_q8", one, 1, 33, None, 0.0, one, one, one, None)
    with pytest.raises(_lib.LeatError, match="null"):
        _lib.call("leat_matvec", 12, None, 4, 256, one, one, one, 1, None, one, None)
    with pytest.raises(_lib.LeatError, match="65 experts a token"):  # a wave holds one slot a lane
        _lib.call("leat_experts_down", 14, one, 128, 4, 512, one, one, one, one, one, 1, 65, None, None, None, one,
                  None)  # fmt: skip


def test_product_path_has_no_cpu_fallback():
    # the kernels refuse CPU tensors rather than computing elsewhere
    import torch

    from leat_amd import _lib, kernels

    with pytest.raises(_lib.LeatError):
        kernels.quantize_q8(torch.zeros(1, 64))


def _parameter_counts() -> dict[str, int]:
    # name -> number of parameters of each function include/leatmi.h declares
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    counts = {}
    for name, params in re.findall(r"\b(leat_\w+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        counts[name] = 0 if params in ("", "void") else params.count(",") + 1
    return counts


def test_binding_argument_counts_match_the_header():
    from leat_amd import _lib

    counts = _parameter_counts()
    for name, args in _lib.SIGNATURES.items():
        assert name in counts, f"{name} is bound but not declared"
        assert len(args) == counts[name], name


def test_attention_workspace_serves_shorter_launches(lib):
    # a workspace for rows of at most L keys serves every launch of fewer keys: its size never
    # shrinks as L grows, although launches of 129..2048 keys take 64-key chunks and longer ones
    # 128-key chunks (2048 keys: 32 chunks, 2049: 17)
    sizes = [lib.leat_attention_workspace(3, 32, n) for n in range(1, 9000, 7)]
    assert all(a <= b for a, b in zip(sizes, sizes[1:]))
    assert lib.leat_attention_workspace(1, 1, 2049) >= lib.leat_attention_workspace(1, 1, 2048)
