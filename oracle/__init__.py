"""CPU oracle of the decode-time KV data plane -- TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker.  The product path (kv_offload_proto_amd) never imports it.
"""
