"""Config surface, mirroring the reference's tests/test_config.py:25-113."""

import pytest
import torch

from sparsetriton_amd.config import (
    ConvAlgo,
    get_conv_algo,
    get_coords_dtype,
    get_h_table_f,
    get_h_table_max_p,
    set_conv_algo,
    set_coords_dtype,
    set_h_table_f,
    set_h_table_max_p,
)


def test_enum_values():
    assert ConvAlgo.ImplicitHashFlyGEMM.value == "Implicit_hashfly_gemm"
    assert ConvAlgo.PrecomputedNeighborGEMM.value == "Precomputed_neighbor_gemm"
    assert len(ConvAlgo) == 2


def test_defaults():
    assert get_coords_dtype() == torch.int16
    assert get_conv_algo() == ConvAlgo.PrecomputedNeighborGEMM
    assert get_h_table_f() == 1.5
    assert get_h_table_max_p() == 16


def test_setters():
    set_coords_dtype(torch.int32)
    assert get_coords_dtype() == torch.int32
    for a in ConvAlgo:
        set_conv_algo(a)
        assert get_conv_algo() == a
    set_h_table_f("3.5")
    assert get_h_table_f() == 3.5
    set_h_table_max_p("64")
    assert get_h_table_max_p() == 64


@pytest.mark.parametrize("bad", ["int32", 32, None])
def test_coords_dtype_type_error(bad):
    with pytest.raises(TypeError):
        set_coords_dtype(bad)


@pytest.mark.parametrize("bad", ["Implicit_hashmap_gemm", 1, None])
def test_algo_type_error(bad):
    with pytest.raises(TypeError):
        set_conv_algo(bad)


@pytest.mark.parametrize("bad", [0.5, 0, -1])
def test_factor_range(bad):
    with pytest.raises(AssertionError, match="factor must be >= 1"):
        set_h_table_f(bad)


@pytest.mark.parametrize("bad", ["not_a_number", None])
def test_factor_type(bad):
    with pytest.raises(TypeError, match="factor must be a number"):
        set_h_table_f(bad)


@pytest.mark.parametrize("bad", [0, -1])
def test_probe_range(bad):
    with pytest.raises(AssertionError, match="probe_n must be positive"):
        set_h_table_max_p(bad)
