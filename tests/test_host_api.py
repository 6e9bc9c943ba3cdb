"""Host-side mirror of the reference module API (CPU): construction, validation errors,
``state_dict`` keys, and the absence of any CPU compute path."""

from __future__ import annotations

import pytest
import torch

from lngram_hip import ops, workloads
from ffnmem.memory import draft, lngram_v2, router, ssm, wrapper

# Keys of the reference module for the SB memory layer (checkpoint compatibility).
SB_KEYS = {
    "module.tables.ngram_2.weight", "module.tables.ngram_3.weight",
    "module.readout_query_norm.weight", "module.readout_memory_norm.weight",
    "module.readout_q_proj.weight", "module.readout_kv_proj.weight", "module.readout_o_proj.weight",
    "module.short_conv.norm.weight", "module.short_conv.conv.weight", "router.weight",
}


def test_state_dict_keys_and_shapes_sb():
    w = workloads.SB
    mem = wrapper.LngramMemory(w.d_model, w.mem_cfg(), 0.02, 1e-5)
    sd = mem.state_dict()
    assert set(sd) == SB_KEYS
    assert sd["module.tables.ngram_2.weight"].shape == (184 * 256, 128)
    assert sd["module.tables.ngram_3.weight"].shape == (184 * 4096, 128)
    assert sd["module.readout_kv_proj.weight"].shape == (512, 256)
    assert sd["module.short_conv.conv.weight"].shape == (1024, 1, 4)
    assert sd["router.weight"].shape == (736, 1024)
    m = mem.module
    assert m.route_token_dim == 256 and m.readout_groups == 4 and m.route_history_length == 2
    assert m.short_conv.left_padding == 9 and abs(m.softmax_scale - 0.125) < 1e-15
    # Appendix E: zero output projection and conv
    assert float(m.readout_o_proj.weight.abs().max()) == 0 and float(m.short_conv.conv.weight.abs().max()) == 0
    assert sum(t.weight.numel() for t in m.tables.values()) == 102_498_304


def test_state_dict_keys_sd_variants():
    mem = wrapper.LngramMemory(64, {"routes": 4, "mem_dim": 16, "kv_heads": 2, "q_heads": 4, "head_dim": 16,
                                    "router_input": "embed2_ssm"}, 0.02, 1e-5, ssm_dim=8)
    keys = set(mem.state_dict())
    assert {"router_features.prev_norm.weight", "router_features.cur_norm.weight", "router_features.start"} <= keys
    assert mem.router.weight.shape == (16, 2 * 64 + 8)
    s = ssm.DiagonalSSM(64, 8, 4)
    assert set(s.state_dict()) == {"norm.weight", "w_in.weight", "theta"}
    a = s.decay()
    assert float(a.min()) >= 0.5 - 1e-6 and float(a.max()) <= 0.999 + 1e-6
    d = draft.DraftReadout(64, mem.module, q_heads=2, head_dim=16, ssm_dim=8)
    assert set(d.state_dict()) == {"q_norm.weight", "w_q.weight", "w_sq.weight", "w_o.weight", "out_norm.weight"}


@pytest.mark.parametrize("kw,msg", [
    (dict(readout_num_heads=3, readout_num_kv_heads=2), "divisible"),
    (dict(readout_num_heads=4, readout_head_dim=8), "full query width"),
    (dict(bits_per_route=0), "bits_per_route"),
    (dict(execution_mode="bogus"), "execution_mode"),
    (dict(ngrams=(0, 2)), "n-gram"),
    (dict(sink_initial_active_mass=1.5), "sink_initial_active_mass"),
])
def test_constructor_validation(kw, msg):
    base = dict(hidden_size=64, num_routes=4, memory_dim=16, readout_num_heads=4, readout_num_kv_heads=2,
                readout_head_dim=16)
    base.update(kw)
    with pytest.raises(ValueError, match=msg):
        lngram_v2.RouteNgramMemoryV2(**base)


def test_router_input_dims_and_errors():
    assert router.router_input_dim("hidden", 1024, 0) == 1024
    assert router.router_input_dim("embed2", 1024, 0) == 2048
    assert router.router_input_dim("embed2_ssm", 1024, 256) == 2304
    with pytest.raises(ValueError):
        router.router_input_dim("embed2_ssm", 1024, 0)
    with pytest.raises(ValueError):
        router.router_input_dim("nope", 1024, 0)


def test_forward_shape_errors_before_any_kernel():
    m = lngram_v2.RouteNgramMemoryV2(64, num_routes=4, memory_dim=16, readout_num_heads=4, readout_num_kv_heads=2,
                                     readout_head_dim=16).eval()
    with pytest.raises(ValueError, match="hidden_states"):
        m(torch.zeros(3, 64), torch.zeros(3, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="hidden size"):
        m(torch.zeros(1, 3, 32), torch.zeros(1, 3, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="incompatible"):
        m(torch.zeros(1, 3, 64), torch.zeros(1, 3, 5, dtype=torch.int32))
    with pytest.raises(ValueError, match="route logits"):
        m.quantize_route_logits(torch.zeros(1, 3, 15))


def test_no_cpu_compute_path():
    m = lngram_v2.RouteNgramMemoryV2(64, num_routes=4, memory_dim=16, readout_num_heads=4, readout_num_kv_heads=2,
                                     readout_head_dim=16).eval()
    with pytest.raises(RuntimeError, match="no CPU path"):
        m(torch.zeros(1, 3, 64), torch.zeros(1, 3, 4, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="no CPU path"):
        ops.ssm_scan(torch.ones(4), torch.zeros(1, 2, 4))
    with pytest.raises(RuntimeError, match="no CPU path"):
        lngram_v2.pack_bits_to_route_codes(torch.zeros(1, 2, 8, dtype=torch.bool), 4)


def test_drafter_shortlist_rules_and_no_cpu_path():
    from drafting.gpu_drafter import GpuDrafter

    cfg, t = workloads.build_draft_bundle(workloads.TINY_DRAFT, seed=0)
    sk = dict(t)
    for n in cfg["ngrams"]:
        sk[f"sketch_ids_{n}"] = torch.zeros(4, 2, dtype=torch.int32)
        sk[f"sketch_counts_{n}"] = torch.ones(4, 2, dtype=torch.int32)
    # the shortlist does not combine with online counts (RefDrafter scores it without them)
    with pytest.raises(ValueError, match="online"):
        GpuDrafter((cfg, sk), shortlist_cap=8, online=True, device="cpu")
    # shortlist or full vocabulary, this host has no GPU path
    for bundle, cap in (((cfg, sk), 8), ((cfg, sk), 0), ((cfg, t), 8)):
        with pytest.raises(RuntimeError, match="no CPU path"):
            GpuDrafter(bundle, shortlist_cap=cap, device="cpu")


def test_storage_dtype_rule():
    assert lngram_v2.route_code_storage_dtype(4) == torch.uint8
    assert lngram_v2.route_code_storage_dtype(12) == torch.int16
    assert lngram_v2.route_code_storage_dtype(16) == torch.int32
    with pytest.raises(ValueError):
        lngram_v2.route_code_storage_dtype(17)


def test_workload_bytes_match_the_roofline_arithmetic():
    # SB: 2 KB h + 2 KB h_norm + 184*2*128*2 rows + 2 KB out = 100,352 B per token
    assert workloads.SB.algorithmic_bytes_per_token() == 100_352
    assert workloads.SB.tokens == 16384


def test_serving_layout_index_helpers_and_no_cpu_path():
    """The serving layout's index bookkeeping (``serving/layout.py:26-35``, ``:84-100``) on the CPU;
    the row movers refuse CPU tensors."""
    import pytest as _pytest
    import torch as _torch

    from serving import layout as sl
    from serving.prefetch import HostGather, LayerTable

    r = sl.reverse_digits(3, 4)
    assert _torch.equal(r[r], _torch.arange(4096))
    assert int(r[1]) == 256 and int(r[16]) == 16 and int(r[0x123]) == 0x321
    hist = _torch.tensor([[[3, 1], [5, 2]]])                     # [B 1, 2 codes, R 2], oldest first
    base = sl.candidate_base(hist, 3, 4)
    assert base.tolist() == [[16 * (5 + 16 * 3), 4096 + 16 * (2 + 16 * 1)]]
    assert LayerTable.num_rows(2, (2, 3), 4) == 2 * (256 + 4096) + 1
    with _pytest.raises(RuntimeError, match="CPU path|ROCm"):
        sl.serving_address(_torch.zeros(1, 4, 2, dtype=_torch.uint8), 2, 4)
    with _pytest.raises(RuntimeError, match="CPU path"):
        HostGather({0: None}, "cpu")
