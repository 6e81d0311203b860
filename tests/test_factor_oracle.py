"""Pins the LoRA-factor storage functions of the CPU oracle (intN dequant, int4
row-pair packing) and the host-side helpers of the checkpoint adapter, on the
CPU.  The reference's own checkpoints are not in this container; the format
is fixed by its writer and loader (cross_layer_share.py:584-649,
inference/model_builder.py:27-80,465-544), restated in the oracle and pinned
here by closed forms and brute force."""

import pytest
import torch

from glorcq_amd import _lib
from glorcq_amd import model_builder as MB
from oracle import glorcq_oracle as O


@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_dequant_intN_closed_forms(nbits):
    maxval = 2 ** (nbits - 1) - 1
    scale = torch.tensor([0.5, 1.25, 3.0]).half()
    q = torch.tensor([[maxval, -maxval, 0]], dtype=torch.int8)
    y = O.dequant_intN(q, scale, nbits)
    assert torch.equal(y, torch.tensor([[0.5, -1.25, 0.0]]).half())


def test_dequant_intN_elementwise_both_layouts():
    g = torch.Generator().manual_seed(0)
    q = torch.randint(-7, 8, (5, 3), generator=g).to(torch.int8)
    col = (torch.rand(3, generator=g) + 0.1).half()
    row = (torch.rand(5, 1, generator=g) + 0.1).half()
    yc, yr = O.dequant_intN(q, col, 4), O.dequant_intN(q, row, 4)
    for r in range(5):
        for c in range(3):
            want_c = torch.tensor(float(q[r, c]), dtype=torch.float32) / 7 * col[c].float()
            want_r = torch.tensor(float(q[r, c]), dtype=torch.float32) / 7 * row[r, 0].float()
            assert yc[r, c] == want_c.half() and yr[r, c] == want_r.half()


def test_int4_every_nibble_both_positions():
    for v in range(-7, 9):  # 8 -> nibble 15, still unpacks to 8
        for pos in range(2):
            packed = torch.zeros(1, 1, dtype=torch.uint8)
            packed[0, 0] = ((v + 7) & 15) << (4 * pos) | (7 << (4 * (1 - pos)))
            got = O.unpack_int4(packed, 2)
            want = torch.zeros(2, 1, dtype=torch.int8)
            want[pos, 0] = v
            assert torch.equal(got, want), (v, pos)


@pytest.mark.parametrize("rows", [1, 4, 7])
def test_int4_round_trip(rows):
    q = torch.randint(-7, 8, (rows, 5), generator=torch.Generator().manual_seed(rows))
    q = q.to(torch.int8)
    assert torch.equal(O.unpack_int4(O.pack_int4(q), rows), q)
    assert torch.equal(MB._unpack_int4(O.pack_int4(q), rows), q)  # host mirror


@pytest.mark.parametrize("nbits,rowwise", [(8, False), (4, False), (4, True), (2, True)])
def test_quant_round_trip_bound(nbits, rowwise):
    t = torch.randn(64, 16, generator=torch.Generator().manual_seed(nbits)) * 0.05
    q, s = O.quant_intN_absmax(t, nbits, rowwise)
    y = O.dequant_intN(q, s, nbits).float()
    maxval = 2 ** (nbits - 1) - 1
    bound = s.float() / (2 * maxval) + 1e-3 * t.abs().max()
    assert bool(((y - t).abs() <= bound).all())


def test_expert_name_helpers():
    """utils/moe_utils.py:9-36 semantics."""
    assert MB.is_regular_expert("mlp.experts.12.gate_proj")
    assert MB.is_regular_expert("block_sparse_moe.experts.3.w1")
    assert not MB.is_regular_expert("mlp.shared_expert.gate_proj")
    assert MB.is_shared_expert("mlp.shared_expert.up_proj")
    assert MB.extract_expert_info("mlp.experts.12.gate_proj") == (12, "gate_proj")
    assert MB.extract_expert_info("experts.0.w2") == (0, "w2")
    assert MB.extract_expert_info("self_attn.q_proj") == (None, None)
    assert MB.module_wtype("block_sparse_moe.experts.3.w2") == "down_proj"
    assert MB.module_wtype("self_attn.o_proj") == "o_proj"
    assert MB.module_expert_index("mlp.shared_expert.gate_proj") == -2
    assert MB.module_expert_index("self_attn.q_proj") == -1


def test_assignment_lookup():
    assignments = {"gate_proj": [{"layer": 0, "expert": 1, "group_id": 3},
                                 {"layer": 1, "expert": 0, "group_id": 3}]}
    lk = MB.build_assignment_lookup(assignments)
    assert lk[("gate_proj", 0, 1)] == (3, "gate_proj", 0)
    assert lk[("gate_proj", 1, 0)] == (3, "gate_proj", 1)


def test_factor_entry_point_checks():
    lib = _lib.load()
    rc = lib.glq_dequant_factor(1 << 12, 1, 4, 4, 1 << 12, 0, 8, 1 << 12, None)
    assert rc == 1 and b"nbits = 4" in lib.glq_last_error()
    rc = lib.glq_dequant_factor(1 << 12, 0, 4, 4, 1 << 12, 0, 9, 1 << 12, None)
    assert rc == 1 and b"nbits" in lib.glq_last_error()
    assert lib.glq_dequant_factor(None, 0, 0, 4, None, 0, 8, None, None) == 0
