"""The HIP library held to the reference's recorded fixtures, through the C ABI (via
dashmag_amd's operations), with the conformance bodies and bounds of crates/dash-conformance."""
import pytest

import conformance as cf
from dashmag_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def adapter():
    from gpu_adapter import GpuAdapter
    return GpuAdapter()


@pytest.mark.parametrize("deterministic", [True, False])
def test_attention_f32(adapter, deterministic):
    worst, compared = cf.matches_torch(adapter, "hip", "f32", deterministic, cf.AUTOTUNE_F32)
    assert compared == 10


@pytest.mark.parametrize("dtype,bounds", [("bf16", cf.BF16), ("f16", cf.F16)])
def test_attention_low_precision(adapter, dtype, bounds):
    worst, compared = cf.matches_torch(adapter, "hip", dtype, True, bounds)
    assert compared == 10


def test_attention_without_gradients(adapter):
    cf.without_gradients(adapter, "hip", cf.AUTOTUNE_F32)


def test_decoding_is_attention_with_one_query(adapter):
    cf.decoding_is_attention_with_one_query(adapter, "hip", [1e-6, 1e-6])


def test_chunk_f32_cases(adapter):
    cf.check_chunk_f32_cases(adapter, "hip")


def test_chunk_bf16_case(adapter):
    """Dk = Dv = 32 in bf16: the MFMA kernels run it (a probe shows it), within the reference's
    tensor-core bound."""
    _lib.probe_reset()
    cf.check_chunk_bf16_case(adapter, "hip", cf.CHUNK_BF16_TC_TOL)
    pc = _lib.probe_counts()
    assert pc["gdr_chunk_fwd_mfma"] > 0 and pc["gdr_chunk_bwd_mfma"] > 0, pc


def test_chunk_packed_f32(adapter):
    cf.check_chunk_packed_f32(adapter, "hip")


def test_chunk_packed_bf16(adapter):
    _lib.probe_reset()
    cf.check_chunk_packed_bf16(adapter, "hip", cf.BF16_TC_VS_F64)
    pc = _lib.probe_counts()
    assert pc["gdr_chunk_fwd_mfma"] > 0 and pc["gdr_chunk_bwd_mfma"] > 0, pc


@pytest.mark.parametrize("name", cf.CHUNK_PACKED_F32)
def test_chunk_packed_equals_per_sequence(adapter, name):
    assert cf.packed_against_sequences(adapter, name, "hip") == cf.PACKED_VS_SEQUENCES


def test_steps(adapter):
    cf.check_steps(adapter, "hip")


def test_f32_steps(adapter):
    cf.check_f32_steps(adapter, "hip")


def test_prefill_then_decode(adapter):
    cf.check_prefill_then_decode(adapter, "hip")


def test_bf16_step(adapter):
    cf.check_bf16_step(adapter, "hip")


def test_step_gradients(adapter):
    """gated_delta_recurrent.rs:229-269: one step's gradients against torch autograd."""
    _lib.probe_reset()
    assert cf.check_gradients(adapter, "hip")
    assert _lib.probe_counts()["gdr_step_bwd"] > 0


def test_packed_step_gradients(adapter):
    """gated_delta_packed.rs:504-517: the packed step's gradients against float64."""
    assert cf.check_step_gradients(adapter, "hip") == 2


def test_default_scale(adapter):
    """gated_delta_packed.rs:519-548."""
    assert cf.the_default_scale_is_one_over_the_root_of_dk(adapter, "hip")
