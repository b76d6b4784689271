"""liboq.so loads, exports every entry point include/oq.h declares, and its host-only registry
functions agree with the oracle (no GPU needed)."""
import ctypes as C
import re
from pathlib import Path

import pytest

import oracle
import oracle_amd
from oracle_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "oq.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(oq_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_bound():
    decl = declared_functions()
    assert len(decl) >= 25
    assert set(decl) == set(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing


def test_registry_matches_oracle():
    for t in range(48):
        got = oracle_amd.ggml_type_layout(t)
        be, bpb, q = C.c_uint64(), C.c_uint64(), C.c_int()
        name = C.c_char_p()
        rc = oracle.lib().orc_type_layout(t, C.byref(be), C.byref(bpb), C.byref(q), C.byref(name))
        if rc != 0:
            assert got is None
        else:
            assert (got.name, got.block_elements, got.bytes_per_block, got.quantized) == \
                (name.value.decode(), be.value, bpb.value, bool(q.value))
        for n in (0, 1, 17, 32, 256, 4096, 12288):
            out = C.c_uint64()
            orc = oracle.lib().orc_row_byte_size(n, t, C.byref(out))
            if orc == 0:
                assert oracle_amd.ggml_row_byte_size(n, t) == out.value
            else:
                with pytest.raises(oracle_amd.OqError) as e:
                    oracle_amd.ggml_row_byte_size(n, t)
                assert e.value.code == orc


def test_known_geometries():
    lay = {t: oracle_amd.ggml_type_layout(t) for t in (8, 12, 14, 15)}
    assert (lay[8].block_elements, lay[8].bytes_per_block) == (32, 34)
    assert (lay[12].block_elements, lay[12].bytes_per_block) == (256, 144)
    assert (lay[14].block_elements, lay[14].bytes_per_block) == (256, 210)
    assert (lay[15].block_elements, lay[15].bytes_per_block) == (256, 292)
    assert oracle_amd.ggml_row_byte_size(4096, 12) == 2304
    assert oracle_amd.ggml_row_byte_size(12288, 12) == 6912
    assert oracle_amd.ggml_row_byte_size(4096, 14) == 3360
    assert oracle_amd.ggml_row_byte_size(4096, 8) == 4352
    assert oracle_amd.ggml_row_byte_size(4096, 15) == 4672
    with pytest.raises(oracle_amd.UnsupportedType):
        oracle_amd.ggml_row_byte_size(255, 12)
    with pytest.raises(oracle_amd.InvalidArgument):
        oracle_amd.ggml_row_byte_size(0, 12)
    assert oracle_amd.ggml_type_layout(4) is None  # deprecated id
    assert oracle_amd.ggml_type_layout(31) is None  # removed id


def test_supported_types():
    assert [t for t in range(48) if oracle_amd.type_supported(t)] == [0, 1, 8, 12, 13, 14, 30]
