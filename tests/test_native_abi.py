"""CPU: the C-ABI library loads and exports every function include/eth_amd.h
declares; argument validation errors surface as ValueError (no GPU calls)."""

import re
from pathlib import Path

import pytest

from eth_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "eth_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(eth_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_functions():
    names = declared_functions()
    assert "eth_bucket_pack" in names and "eth_adam_step" in names
    assert len(names) >= 8


def test_library_exports_every_declared_symbol():
    lib = nat.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in eth_amd.h but not exported"
    assert set(declared_functions()) == set(nat.exported_symbols())
    assert lib.eth_abi_version() >= 1


def test_integration_guide_names_every_declared_symbol():
    """The binding guide's export table keeps up with the header: a
    maintainer binding the reference finds every function there."""
    guide = (HEADER.parents[1] / "INTEGRATION.md").read_text()
    missing = [name for name in declared_functions() if f"`{name}`" not in guide]
    assert not missing, f"not in the integration guide: {missing}"


def test_invalid_arguments_raise_value_error_without_gpu():
    with pytest.raises(ValueError, match="unsupported dtype"):
        nat.call("eth_bucket_pack", None, 1, None, 9, None)
    with pytest.raises(ValueError, match="step must be positive"):
        nat.call("eth_adam_step", None, None, 1, 0.9, 0.999, 1e-8, 0, nat.ETH_BF16, None, None, None)
    with pytest.raises(ValueError, match="unscale requires fp32"):
        nat.call("eth_bucket_unpack", None, 1, None, nat.ETH_BF16, 1.0, 0.5, nat.UNPACK_UNSCALE, None, None, 0, None)


def test_struct_layouts_match_header():
    assert nat.CHUNK_DTYPE.itemsize == 40
    assert nat.ADAM_TENSOR_DTYPE.itemsize == 64
    assert nat.ADAM_CHUNK_DTYPE.itemsize == 16
    text = HEADER.read_text()
    assert f"#define ETH_CHUNK_ELEMS {nat.CHUNK_ELEMS}" in text
