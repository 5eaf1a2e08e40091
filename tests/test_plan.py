"""CPU: the split planner and kernel choice behind tq_sdpa_int4_plan (host
code only; no GPU call).  The kernel a call launches is part of the
contract the bench and the GPU tests rely on: the reference's own cache
dtype (fp32 scale/bias, lib/turboquant.h:199) must reach the matrix-core
kernel like fp16 does."""
import pytest
import torch

from gemma4metal_amd import turboquant as tq

F16, F32 = torch.float16, torch.float32


def test_headline_plan():
    pl = tq.sdpa_plan(32, 16, 256, 32768)
    assert pl == {"kernel": "sdpa_int4_mfma_kernel", "splits": 16, "chunk": 2048}


@pytest.mark.parametrize("sb", [F16, F32])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 16, 256), (2, 1, 128), (16, 2, 128), (32, 8, 256),
                                      (8, 4, 512), (8, 8, 512), (12, 4, 512)])
def test_matrix_core_kernel_for_both_scale_dtypes(Hq, Hkv, D, sb):
    assert tq.sdpa_plan(Hq, Hkv, D, 5000, sb_dtype=sb)["kernel"] == "sdpa_int4_mfma_kernel"


@pytest.mark.parametrize("sb", [F16, F32])
def test_global_layer_kernels(sb):
    # D 512 with GQA 8 (Gemma global layers): the wave-specialised
    # heads-as-columns kernel for both scale/bias dtypes
    assert tq.sdpa_plan(32, 4, 512, 32768, sb_dtype=sb)["kernel"] == "sdpa_int4_hc2_kernel"
    assert tq.sdpa_plan(32, 2, 512, 5000, sb_dtype=sb)["kernel"] == "sdpa_int4_hc2_kernel"


def test_one_wave_global_kernel_is_fp16_only(tq_env):
    tq_env("TQ_HC_IMPL", "1")
    assert tq.sdpa_plan(32, 4, 512, 32768)["kernel"] == "sdpa_int4_hc_kernel"
    # fp32 scale/bias: the matrix-core kernel, two heads per workgroup
    assert tq.sdpa_plan(32, 4, 512, 32768, sb_dtype=F32)["kernel"] == "sdpa_int4_mfma_kernel"


def test_odd_gqa_and_forced_valu(tq_env):
    assert tq.sdpa_plan(12, 4, 512, 3000)["kernel"] == "sdpa_int4_mfma_kernel"  # GQA 3, D 512
    assert tq.sdpa_plan(32, 4, 256, 3000)["kernel"] == "sdpa_int4_mfma_kernel"  # GQA 8, D 256
    tq_env("TQ_SDPA_IMPL", "valu")
    assert tq.sdpa_plan(32, 16, 256, 32768)["kernel"] == "sdpa_int4_kernel"


def test_forced_chunk_and_reload(tq_env):
    tq_env("TQ_SDPA_CHUNK", "1024")
    assert tq.sdpa_plan(32, 16, 256, 32768)["chunk"] == 1024
    assert tq.sdpa_plan(32, 16, 256, 32768)["splits"] == 32


def test_switches_restored_after_fixture():
    # the tq_env fixture of the previous tests restored the environment and
    # re-read the switches
    assert tq.sdpa_plan(32, 16, 256, 32768)["chunk"] == 2048


def test_sliding_and_prefill_plans():
    sl = tq.sdpa_plan(32, 16, 256, 786, sliding_window=1024)
    assert sl["kernel"] == "sdpa_int4_mfma_kernel" and sl["splits"] * sl["chunk"] >= 786
    pf = tq.sdpa_plan(32, 16, 256, 4096, mode="prefill", batch=512, sliding_window=1024)
    assert pf["kernel"] == "prefill_int4_ws_kernel"
    pf32 = tq.sdpa_plan(32, 16, 256, 4096, mode="prefill", batch=512, sb_dtype=F32)
    assert pf32["kernel"] == "prefill_int4_ws_kernel"
    g32 = tq.sdpa_plan(32, 4, 512, 4096, mode="prefill", batch=512, sb_dtype=F32)
    assert g32["kernel"] == "prefill_int4_kernel"


def test_plan_rejects_bad_arguments():
    from gemma4metal_amd._lib import TQError
    with pytest.raises(TQError):
        tq.sdpa_plan(32, 16, 96, 100)
    with pytest.raises(TQError):
        tq.sdpa_plan(30, 16, 256, 100)


def test_ragged_plan_bounds_the_device_chunk():
    # ragged batches of up to 64 sequences choose their chunk on the device
    # (1 .. splits chunks of the longest); with >= 2 (sequence, head) jobs
    # per CU the grid allows at most two
    pl = tq.sdpa_plan(32, 16, 256, 32769, mode="ragged", batch=64)
    assert pl["splits"] == 2 and pl["chunk"] >= (32769 + 1) // 2
    small = tq.sdpa_plan(32, 16, 256, 32769, mode="ragged", batch=8)
    assert small["splits"] == 5
