"""The decode driver's host pieces, without a GPU: flags and defaults of the
reference driver (xds/xds_decode.py:21-45), the row fingerprint
(xds_decode.py:60-63) against its closed form in Python integers, and the
driver's CPU SIEVE model (used by --oracle) against the C oracle."""
import numpy as np
import pytest
import torch

from kv_offload_proto_amd.xds import streams, xds_decode
from oracle import oracle as orc


def _word(row, layer, k):
    """The reference formula, in Python's unbounded integers."""
    P1, P2, M1, M2 = 0x9E3779B1, 0x85EBCA77, 0x27220A95, 0x165667B1
    v = (row * P1 + layer * P2) * M1 ^ M2
    return (v + k * M1) & 0xFFFFFFFF


def test_flags_and_defaults_follow_the_reference():
    a = xds_decode.parse_args([])
    ref = dict(device=0, layers=2, kv_lora_rank=512, qk_rope=64, stripe_rows=1, req_num=8, prefill=256, topk=64,
               device_buffer_size=64, miss_ratio=0.5, steps=10, seed=42, block_dim=8, oracle=False,
               run_dir="./log", rootinfo="/etc/hccl_rootinfo.json", fatbin="")
    for k, v in ref.items():
        assert getattr(a, k) == v, k
    a = xds_decode.parse_args(["--ems-master", "10.0.0.1:9000", "--oracle", "--layers", "3"])
    assert a.ems_master == "10.0.0.1:9000" and a.oracle and a.layers == 3


@pytest.mark.parametrize("layer", [0, 1, 60])
def test_fingerprint_matches_closed_form(layer):
    rows = np.array([0, 1, 255, 4096, 524287, 2**31 - 1, 2**32 - 1], dtype=np.int64)
    got = xds_decode.fingerprint_rows(torch, torch.from_numpy(rows), layer, 288).numpy().view(np.uint32)
    for i, r in enumerate(rows):
        for k in (0, 1, 7, 143, 287):
            assert int(got[i, k]) == _word(int(r), layer, k), (r, k)


@pytest.mark.parametrize("dbs,prefill,top_k,miss", [(64, 256, 64, 0.5), (16, 40, 30, 0.8), (100, 1000, 64, 0.2)])
def test_cpu_model_matches_oracle(dbs, prefill, top_k, miss):
    """Slots and is_miss of the driver's model equal the C oracle's over
    streams that wrap the hand, repeat tokens and include invalid and
    decode-extension positions."""
    R, L = 6, 1
    st = orc.SieveState(L, R, dbs, top_k)
    for r in range(R):
        st.admit(r, prefill)
    models = [xds_decode.CpuSieve(prefill, dbs, st.padded) for _ in range(R)]
    rng = np.random.default_rng(dbs + top_k)
    seq = np.full(R, prefill + 8, dtype=np.int32)
    for step in range(12):
        if step % 2:
            batch = streams.ref_batch(rng, R, top_k, prefill, dbs, miss)
        else:
            batch = rng.integers(-3, prefill + 10, size=(R, top_k)).astype(np.int32)
        e_slots, e_miss = st.update(0, batch, np.arange(R), seq, R)
        for r in range(R):
            s, m = models[r].update(batch[r], int(seq[r]))
            np.testing.assert_array_equal(m, e_miss[r], err_msg="step {} req {}".format(step, r))
            np.testing.assert_array_equal(s, e_slots[r], err_msg="step {} req {}".format(step, r))
