"""The C ABI library loads without a GPU and exports every function include/msx.h declares;
its device-free entry points behave."""
import os
import re

import pytest

from modelspec_amd import api

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "msx.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(msx_[a-z_0-9]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 18
    lib = api.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_compile_rejects_an_unknown_config():
    with pytest.raises(api.MsxError, match="unknown config"):
        api.compile_config("no_such_model")


def test_check_ir_rejects_malformed_text():
    with pytest.raises(api.MsxError):
        api.check_ir("forward %0: Tensor<f32, [2]> = Bogus %7\n")
    with pytest.raises(api.MsxError, match="before its definition"):
        api.check_ir("%0: Tensor<f32, [2]> = Relu %1\n%1: Tensor<f32, [2]> = Input \"x\"\noutput %0\n")


def test_check_ir_rejects_a_mistyped_node():
    text = "%0: Tensor<f32, [2, 3]> = Input \"a\"\n%1: Tensor<f32, [3, 4]> = Input \"b\"\n" \
           "%2: Tensor<f32, [2, 5]> = MatMul %0, %1\noutput %2\n"
    with pytest.raises(api.MsxError, match="types as"):
        api.check_ir(text)
