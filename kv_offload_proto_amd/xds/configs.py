"""The five benchmark/parity workloads of the decode-time KV data plane.

Shapes follow the reference driver's flags (xds/xds_decode.py:21-45) and the
row format of an MLA latent row: (kv_lora_rank 512 + qk_rope 64) fp16 =
1152 bytes, 128-byte aligned (xds_decode.py:126-127).
"""
from dataclasses import dataclass, field
from typing import Optional


def row_bytes_of(kv_lora_rank=512, qk_rope=64, elem_bytes=2):
    return -(-((kv_lora_rank + qk_rope) * elem_bytes) // 128) * 128


@dataclass
class Workload:
    name: str
    req_num: int
    prefill: int
    top_k: int
    dbs: int
    miss_ratio: float
    layers: int
    node_num: int
    stripe_rows: int
    steps: int
    seed: int
    stream: str = "state"          # "ref" (reference driver stream) or "state"
    zipf_s: Optional[float] = None
    adversarial: bool = False
    # adversarial misses come from the positions whose 16-bit Knuth hash is
    # below this bound (their homes share one window of the table); the pool
    # must hold more than dbs + miss_ratio*topK positions, or it runs dry once
    # the buffer is full of them
    adversarial_hash_below: int = 40960
    export_reqs: Optional[int] = None   # prefill requests exported (default req_num)
    row_bytes: int = field(default_factory=row_bytes_of)

    @property
    def host_reqs(self):
        return self.export_reqs if self.export_reqs is not None else self.req_num

    @property
    def layer_rows(self):
        # The reference default layer_rows=1024 cannot hold req*prefill rows
        # (xds_decode.py:29-30,173); every workload sizes it to fit.
        return self.host_reqs * self.prefill

    @property
    def padded(self):
        return -(-self.dbs // 16) * 16

    @property
    def rows_per_layer_step(self):
        return self.req_num * self.top_k


CONFIGS = {
    # reference default shape, CPU oracle
    0: Workload("c0-cpu-default", req_num=8, prefill=256, top_k=64, dbs=64, miss_ratio=0.5, layers=2, node_num=2,
                stripe_rows=1, steps=10, seed=42),
    # same stream and shapes through the HIP kernels
    1: Workload("c1-hip-default", req_num=8, prefill=256, top_k=64, dbs=64, miss_ratio=0.5, layers=2, node_num=2,
                stripe_rows=1, steps=10, seed=42),
    # DSA-decode scale
    2: Workload("c2-dsa-decode", req_num=64, prefill=8192, top_k=2048, dbs=4096, miss_ratio=0.2, layers=61,
                node_num=4, stripe_rows=1, steps=20, seed=7, zipf_s=1.1),
    # large batch after a striped prefill export
    3: Workload("c3-large-batch-export", req_num=256, prefill=16384, top_k=2048, dbs=8192, miss_ratio=0.1,
                layers=61, node_num=4, stripe_rows=64, steps=10, seed=11, export_reqs=16),
    # SIEVE stress at the uint16 slot limit, adversarial hash collisions: the
    # misses come from the 81,922 positions below 131,072 whose hash is below
    # 40,960 (more than dbs + 0.9*topK = 72,891), so every step has ~7,400
    # misses per request inside one long probe run
    4: Workload("c4-slot-limit-stress", req_num=4, prefill=131072, top_k=8192, dbs=65518, miss_ratio=0.9, layers=4,
                node_num=2, stripe_rows=1, steps=50, seed=3, adversarial=True),
}
