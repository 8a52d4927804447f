"""GPU parity of the SIEVE kernels against the C oracle: slots, is_miss and
the full state (tokens, visited, hand, hash table) after every launch."""
import numpy as np
import pytest

from gpu_helpers import DevSieve, to_dev
from kv_offload_proto_amd.xds import streams
from kv_offload_proto_amd.xds.configs import CONFIGS
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _admit_all(st, cfg):
    for r in range(cfg.req_num):
        st.admit(r, cfg.prefill)


def test_ht_init_parity(kvops):
    import torch

    rng = np.random.default_rng(11)
    layers, pool, dbs, top_k = 3, 5, 300, 64
    st = orc.SieveState(layers, pool, dbs, top_k)
    st.tokens[:] = -1
    for l in range(layers):
        for r in range(pool):
            n = int(rng.integers(0, dbs + 1))
            st.tokens[l, r, :n] = rng.choice(50000, size=n, replace=False)
    dev = DevSieve(st)
    dev.ht.fill_(77)
    orc.sieve_ht_init(st.tokens, st.ht, 0, pool, layers, pool, dbs, st.padded, st.ht_size)
    kvops.sieve_ht_init(dev.tokens.data_ptr(), dev.ht.data_ptr(), dev.prefill.data_ptr(), 0, pool, layers, pool,
                        dbs, st.padded, st.ht_size, 0, layers)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dev.ht.cpu().numpy().view(np.uint16), st.ht)
    assert kvops.read_overflow() == 0


def _home(t, ht_size):
    return ((np.asarray(t, dtype=np.uint64) * 2654435761) & 0xFFFFFFFF) >> 16 & (ht_size - 1)


def _ht_rows(rng, st, mode):
    """Token rows for the admission build: 'unique', 'dups' (duplicates and
    negatives), 'few_homes' (all keys on 8 home cells: long clusters) or
    'wrap' (homes in the last 40 cells: clusters across the table's end)."""
    L, R = st.tokens.shape[:2]
    H = st.ht_size
    st.tokens[:] = -1
    cand = None
    if mode in ("few_homes", "wrap"):
        t = np.arange(0, 1 << 23, dtype=np.int64)
        h = _home(t, H)
        if mode == "few_homes":
            homes = rng.choice(H, size=8, replace=False)
            cand = t[np.isin(h, homes)]
        else:
            cand = t[h >= H - 40]
    for l in range(L):
        for r in range(R):
            n = int(rng.integers(0, st.dbs + 1))
            if mode == "unique":
                vals = rng.choice(1 << 22, size=n, replace=False)
            elif mode == "dups":
                vals = rng.integers(-3, max(4, n // 3), size=n)
            else:
                n = min(n, len(cand), st.ht_size // 16)
                vals = rng.choice(cand, size=n, replace=False)
            slots = rng.choice(st.dbs, size=n, replace=False)
            st.tokens[l, r, slots] = vals


@pytest.mark.parametrize("mode", ["unique", "dups", "few_homes", "wrap"])
@pytest.mark.parametrize("dbs,top_k", [(4096, 2048), (8192, 2048)])
def test_ht_init_parallel_parity(kvops, dbs, top_k, mode):
    """The admission build at the DSA-decode and large-batch table sizes
    (16384 and 32768 cells, the parallel form): every table byte equals the
    oracle's sequential inserts, rows outside [req_start, req_start+num_reqs)
    untouched."""
    import torch

    rng = np.random.default_rng(dbs + len(mode))
    layers, pool = 2, 3
    st = orc.SieveState(layers, pool, dbs, top_k)
    _ht_rows(rng, st, mode)
    dev = DevSieve(st)
    dev.ht.fill_(77)
    st.ht[:] = 77
    orc.sieve_ht_init(st.tokens, st.ht, 1, 2, layers, pool, dbs, st.padded, st.ht_size)
    kvops.sieve_ht_init(dev.tokens.data_ptr(), dev.ht.data_ptr(), dev.prefill.data_ptr(), 1, 2, layers, pool,
                        dbs, st.padded, st.ht_size, 0, 0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dev.ht.cpu().numpy().view(np.uint16), st.ht)
    assert kvops.read_overflow() == 0


def _wave_rows(rng, st, mode):
    """Token rows for tables past the parallel form's LDS budget: 'identity'
    (slot s holds token s, the admission pattern), 'spread' (distinct tokens
    below 2^20), 'dense' (distinct tokens homed in the lowest quarter: long
    clusters), 'wrap' (homes in the last 64 cells: clusters across the end),
    'dups' (repeated tokens) and 'big' (one token at 2^20 or above); the last
    two take the one-lane inserts."""
    L, R = st.tokens.shape[:2]
    H, dbs = st.ht_size, st.dbs
    st.tokens[:] = -1
    t = np.arange(0, 1 << 20, dtype=np.int64)
    h = _home(t, H)
    cand = {"spread": t, "dense": t[h < H // 4], "wrap": t[h >= H - 64], "big": t, "dups": t}.get(mode)
    for l in range(L):
        for r in range(R):
            n = int(rng.integers(dbs // 2, dbs + 1))
            if mode == "identity":
                st.tokens[l, r, :n] = np.arange(n)
                continue
            n = min(n, len(cand))
            vals = rng.choice(cand, size=n, replace=False)
            if mode == "dups" and n > 8:
                vals[rng.integers(0, n, size=n // 8)] = vals[rng.integers(0, n, size=n // 8)]
            if mode == "big" and n > 0:
                vals[rng.integers(0, n)] = (1 << 20) + int(rng.integers(0, 1000))
            st.tokens[l, r, rng.choice(dbs, size=n, replace=False)] = vals


@pytest.mark.parametrize("mode", ["identity", "spread", "dense", "wrap", "dups", "big"])
@pytest.mark.parametrize("dbs,top_k", [(16000, 2048), (32768, 2048), (65518, 8192)])
def test_ht_init_wave_parity(kvops, dbs, top_k, mode):
    """The admission build for tables past the parallel form's LDS budget
    (65536, 131072 and 262144 cells: the batched wave build, or the one-lane
    inserts for repeated or large tokens): every table byte equals the
    oracle's sequential inserts, rows outside [req_start, req_start+num_reqs)
    untouched."""
    import torch

    if mode == "wrap" and dbs != 16000:
        pytest.skip("homes reach the table's end only in a 65536-cell table")
    print("ht_init wave case", dbs, top_k, mode, flush=True)
    rng = np.random.default_rng(dbs + 7 * len(mode))
    layers, pool = 2, 3
    st = orc.SieveState(layers, pool, dbs, top_k)
    _wave_rows(rng, st, mode)
    dev = DevSieve(st)
    dev.ht.fill_(77)
    st.ht[:] = 77
    orc.sieve_ht_init(st.tokens, st.ht, 1, 2, layers, pool, dbs, st.padded, st.ht_size)
    kvops.sieve_ht_init(dev.tokens.data_ptr(), dev.ht.data_ptr(), dev.prefill.data_ptr(), 1, 2, layers, pool,
                        dbs, st.padded, st.ht_size, 0, 0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dev.ht.cpu().numpy().view(np.uint16), st.ht)
    assert kvops.read_overflow() == 0


def test_ht_init_small_table_parity(kvops):
    """A 512-cell table (under the parallel form's 1024): the one-lane build."""
    import torch

    rng = np.random.default_rng(5)
    layers, pool, dbs = 2, 4, 200
    st = orc.SieveState(layers, pool, dbs, 8)
    _ht_rows(rng, st, "dups")
    ht_size = 512
    dev = DevSieve(st)
    want = np.full((layers, pool, ht_size), 77, dtype=np.uint16)
    got = torch.full((layers, pool, ht_size), 77, dtype=torch.int16, device="cuda")
    orc.sieve_ht_init(st.tokens, want, 0, pool, layers, pool, dbs, st.padded, ht_size)
    kvops.sieve_ht_init(dev.tokens.data_ptr(), got.data_ptr(), dev.prefill.data_ptr(), 0, pool, layers, pool,
                        dbs, st.padded, ht_size, 0, 0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), want)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("cfg_id", [0, 1])
def test_sieve_ref_stream_parity(kvops, cfg_id):
    """The reference driver's stream (xds_decode.py:211-225): one layer per step."""
    cfg = CONFIGS[cfg_id]
    st = orc.SieveState(cfg.layers, cfg.req_num, cfg.dbs, cfg.top_k)
    _admit_all(st, cfg)
    dev = DevSieve(st)
    rng = np.random.default_rng(cfg.seed)
    req_pool = np.arange(cfg.req_num)
    seq = np.full(cfg.req_num, cfg.prefill)
    for step in range(cfg.steps):
        batch = streams.ref_batch(rng, cfg.req_num, cfg.top_k, cfg.prefill, cfg.dbs, cfg.miss_ratio)
        layer = step % cfg.layers
        e_slots, e_miss = st.update(layer, batch, req_pool, seq, cfg.req_num)
        g_slots, g_miss, _ = dev.update(kvops, layer, batch, req_pool, seq, cfg.req_num, cfg.req_num, cfg.top_k)
        np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
        np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
        dev.assert_state_equal(layer)
    assert kvops.read_overflow() == 0


def test_sieve_state_stream_parity_all_layers(kvops):
    """config 1 shapes, state-driven stream (~50% non-resident), every layer every step."""
    cfg = CONFIGS[1]
    st = orc.SieveState(cfg.layers, cfg.req_num, cfg.dbs, cfg.top_k)
    _admit_all(st, cfg)
    dev = DevSieve(st)
    rng = np.random.default_rng(cfg.seed)
    req_pool = np.arange(cfg.req_num)
    seq = np.full(cfg.req_num, cfg.prefill)
    for step in range(cfg.steps):
        for layer in range(cfg.layers):
            batch = streams.state_batch(rng, st.tokens[layer, :cfg.req_num, :cfg.dbs], cfg.prefill, cfg.top_k,
                                        cfg.miss_ratio)
            e_slots, e_miss = st.update(layer, batch, req_pool, seq, cfg.req_num)
            g_slots, g_miss, _ = dev.update(kvops, layer, batch, req_pool, seq, cfg.req_num, cfg.req_num, cfg.top_k)
            np.testing.assert_array_equal(g_miss, e_miss)
            np.testing.assert_array_equal(g_slots, e_slots)
    dev.assert_state_equal()


@pytest.mark.parametrize("variant", [-1, 2, 3, 5])
@pytest.mark.parametrize("seed", range(6))
def test_sieve_defensive_cases_parity(kvops, seed, variant):
    """Padding rows, out-of-range pool rows, num_real > max, dirty hands,
    invalid and decode-extension positions, duplicates, tiny buffers (wrap);
    automatic variant, the wave-wide HBM kernel and the batch HBM kernel
    (whose wrapping rows take its in-order path)."""
    rng = np.random.default_rng(500 + seed)
    dbs = int(rng.integers(1, 70))
    top_k = int(rng.integers(1, 90))
    pool, max_reqs = 6, 7
    st = orc.SieveState(1, pool, dbs, top_k)
    prefills = [int(rng.integers(1, 4 * dbs + 8)) for _ in range(pool)]
    for r in range(pool):
        st.admit(r, prefills[r])
    st.hand[0, 1, 0] = dbs + 3
    dev = DevSieve(st)
    kvops.sieve_force_variant(variant)
    try:
        _defensive_steps(kvops, rng, st, dev, pool, max_reqs, prefills, top_k, seed)
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


def _defensive_steps(kvops, rng, st, dev, pool, max_reqs, prefills, top_k, seed):
    for step in range(5):
        rows = list(rng.permutation(pool))[: int(rng.integers(1, pool + 1))]
        req_pool = rows + [-1] * (max_reqs - len(rows))
        req_pool[int(rng.integers(max_reqs))] = int(rng.choice([-4, pool, pool + 9]))
        seen = set()
        for i, p in enumerate(req_pool):
            if 0 <= p < pool:
                if p in seen:
                    req_pool[i] = -1
                seen.add(p)
        num_real = int(rng.integers(0, max_reqs + 3))
        seq = [int((prefills[p] if 0 <= p < pool else 5) + rng.integers(-3, 6)) for p in req_pool]
        topk = np.stack([rng.integers(-3, max(s + 4, 2), size=top_k) for s in seq]).astype(np.int32)
        e_slots, e_miss = st.update(0, topk, req_pool, seq, num_real, max_num_reqs=max_reqs)
        g_slots, g_miss, _ = dev.update(kvops, 0, topk, req_pool, seq, num_real, max_reqs, top_k)
        np.testing.assert_array_equal(g_miss, e_miss, err_msg="seed {} step {}".format(seed, step))
        np.testing.assert_array_equal(g_slots, e_slots, err_msg="seed {} step {}".format(seed, step))
        dev.assert_state_equal()


def test_sieve_validation_messages(kvops):
    base = dict(topk_indices=0, req_pool_indices=0, seq_lens=0, prefill_lens=0, device_buffer_tokens=0,
                device_buffer_visited=0, device_buffer_ht=0, sieve_hand=0, topk_device_slots=0, is_miss=0,
                num_real=0, top_k=8, device_buffer_size=16, padded_buffer_size=16, visited_stride_b=64,
                max_num_reqs=0, pool_size=1)
    cases = [
        (dict(padded_buffer_size=24), "padded_buffer_size must be a multiple of 16"),
        (dict(padded_buffer_size=65536, device_buffer_size=65536), "padded_buffer_size must be <= 65534"),
        (dict(visited_stride_b=32), "visited bitmap stride must be 64B aligned"),
        (dict(padded_buffer_size=1024, device_buffer_size=1024, visited_stride_b=64),
         "visited bitmap stride must be 64B aligned and cover padded"),
    ]
    for over, msg in cases:
        kw = dict(base)
        kw.update(over)
        with pytest.raises(RuntimeError, match=msg):
            kvops.sieve_update(**kw)
    kvops.sieve_update(**base)  # max_num_reqs == 0: nothing to launch


def _random_state_stream(rng, st, K, prefill, seq_extra=4, miss_frac=None):
    """Mixed batch like the fast-path fuzz: resident hits in random order,
    non-resident misses, a few invalid/extension positions and duplicates."""
    req = st.pool_size
    miss_frac = rng.random() if miss_frac is None else miss_frac
    out = np.empty((req, K), dtype=np.int32)
    for r in range(req):
        tok = st.tokens[0, r, :st.dbs]
        res = tok[tok >= 0]
        row = np.where(rng.random(K) < miss_frac, rng.integers(0, prefill, K),
                       res[rng.integers(0, len(res), K)] if len(res) else rng.integers(0, prefill, K))
        junk = rng.random(K) < 0.03
        row[junk] = rng.integers(-3, prefill + seq_extra + 3, junk.sum())
        dup = rng.random(K) < 0.05
        row[dup] = row[rng.integers(0, K, dup.sum())]
        out[r] = row
    return out


@pytest.mark.parametrize("seed", range(8))
def test_sieve_fast_kernel_parity_mid(kvops, seed):
    """The parallel kernel (variant 2) at mid sizes with conversion-heavy
    streams: full state, including the exact table layout, after every step."""
    rng = np.random.default_rng(900 + seed)
    dbs = int(rng.integers(300, 1500))
    K = int(rng.integers(64, 700))
    prefill = dbs + int(rng.integers(1, 4000))
    req = 6
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    variants = set()
    for step in range(6):
        batch = _random_state_stream(rng, st, K, prefill)
        seq = np.full(req, prefill + 2)
        e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
        g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
        variants.add(kvops.last_sieve_variant())
        np.testing.assert_array_equal(g_miss, e_miss, err_msg="seed {} step {}".format(seed, step))
        np.testing.assert_array_equal(g_slots, e_slots, err_msg="seed {} step {}".format(seed, step))
        dev.assert_state_equal()
    assert variants == {2}
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("dbs,top_k,prefill", [(4096, 2048, 6000), (4096, 1500, 9000), (4096, 2048, 60000),
                                               (3500, 1100, 7000), (8192, 2048, 12000), (8192, 1300, 50000)])
def test_sieve_fixed_kernels_mixed_streams(kvops, dbs, top_k, prefill):
    """The fixed-count kernels (two positions per lane, four or eight ring
    offsets) on streams with duplicate positions, invalid and decode-extension
    positions and a random miss share per step; topK below 2048 leaves the
    upper lanes' second position past topK; a prefill above the direct map's
    capacity takes the probing classify; 8192 slots take the compact form."""
    req = 6
    st = orc.SieveState(1, req, dbs, top_k)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    rng = np.random.default_rng(dbs + top_k + prefill)
    parallel = 0
    for step in range(5):
        # miss shares the hand can serve without coming round (else the row
        # takes the in-order recurrence for the next steps)
        batch = _random_state_stream(rng, st, top_k, prefill, miss_frac=float(rng.uniform(0.05, 0.3)))
        seq = np.full(req, prefill + 2)
        e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
        g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, top_k)
        assert kvops.last_sieve_variant() == (4 if dbs > 4096 else 2)
        np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
        np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
        dev.assert_state_equal()
        # sieve_hand[row][2] counts the steps in a row taken in order: 0 after a parallel one
        parallel += int((dev.hand[0, :, 2].cpu().numpy() == 0).sum())
    assert parallel >= 5 * req // 2
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("dbs", [4096, 8192])
def test_sieve_fast_kernel_shuffled_batch(kvops, dbs):
    """The fixed-count kernels (topK 2048; rings of 4096 slots in the full LDS
    form, 8192 in the compact one) on
    batches whose rows are not their pool rows: 32 of 40 requests in a new
    random order each step, about a quarter of them at their own index, each
    with its own prefill length, plus rows past num_real."""
    top_k, pool, batch_n, max_reqs = 2048, 40, 32, 36
    st = orc.SieveState(1, pool, dbs, top_k)
    rng = np.random.default_rng(dbs + 5)
    prefills = [int(rng.integers(dbs // 2, 3 * dbs)) for _ in range(pool)]
    for r in range(pool):
        st.admit(r, prefills[r])
    dev = DevSieve(st)
    for step in range(4):
        perm = [int(x) for x in rng.permutation(pool)[:batch_n]]
        for i in range(batch_n):
            if rng.random() < 0.25 and i in perm:
                j = perm.index(i)
                perm[i], perm[j] = perm[j], perm[i]
        assert perm != list(range(batch_n))
        req_pool = perm + [int(x) for x in rng.integers(0, pool, size=max_reqs - batch_n)]
        seq = [prefills[p] + step for p in req_pool]
        batch = np.stack([streams.state_batch(rng, st.tokens[0, p:p + 1, :dbs], prefills[p], top_k, 0.2)[0]
                          for p in req_pool]).astype(np.int32)
        e_slots, e_miss = st.update(0, batch, req_pool, seq, batch_n, max_num_reqs=max_reqs)
        g_slots, g_miss, _ = dev.update(kvops, 0, batch, req_pool, seq, batch_n, max_reqs, top_k)
        assert kvops.last_sieve_variant() == (2 if dbs == 4096 else 4)  # 8192 slots: the compact LDS form
        np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
        np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
        dev.assert_state_equal()
    assert kvops.read_overflow() == 0


def test_sieve_fast_kernel_parity_dsa_scale(kvops):
    """DSA-decode shapes (64 requests, topK 2048, 4096 slots, Zipf recency
    hits, 20% misses) over two layers and three steps."""
    from kv_offload_proto_amd.xds.configs import CONFIGS

    cfg = CONFIGS[2]
    L = 2
    st = orc.SieveState(L, cfg.req_num, cfg.dbs, cfg.top_k)
    for r in range(cfg.req_num):
        st.admit(r, cfg.prefill)
    dev = DevSieve(st)
    rng = np.random.default_rng(cfg.seed)
    req_pool = np.arange(cfg.req_num)
    seq = np.full(cfg.req_num, cfg.prefill)
    for step in range(3):
        for layer in range(L):
            batch = streams.state_batch(rng, st.tokens[layer, :, :cfg.dbs], cfg.prefill, cfg.top_k, cfg.miss_ratio,
                                        zipf_s=cfg.zipf_s)
            e_slots, e_miss = st.update(layer, batch, req_pool, seq, cfg.req_num)
            g_slots, g_miss, _ = dev.update(kvops, layer, batch, req_pool, seq, cfg.req_num, cfg.req_num, cfg.top_k)
            assert kvops.last_sieve_variant() == 2
            np.testing.assert_array_equal(g_miss, e_miss)
            np.testing.assert_array_equal(g_slots, e_slots)
        dev.assert_state_equal()
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("K,dbs,force", [(2048, 4096, 4), (2500, 3000, -1), (1500, 6000, -1), (1024, 8192, -1),
                                         (2048, 8192, 4), (64, 4096, -1)])
def test_sieve_parallel_kernel_shapes(kvops, K, dbs, force):
    """The parallel kernel's instantiations: positions and ring offsets per
    lane fixed at (2, 4) / (2, 8), or any shape (P = ceil(topK/1024), Q =
    ceil(dbs/1024) of 1..8), in the full and the compact LDS form."""
    rng = np.random.default_rng(K * 7 + dbs)
    prefill, req = dbs + 5000, 8
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(force)
    variants = set()
    try:
        for step in range(4):
            batch = _random_state_stream(rng, st, K, prefill)
            seq = np.full(req, prefill + 3)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            variants.add(kvops.last_sieve_variant())
            np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
            np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert variants <= {2, 4} and len(variants) == 1
    if force == 4:
        assert variants == {4}
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5])
def test_sieve_variants_agree(kvops, variant):
    """Sequential LDS (0), single-lane HBM (1), parallel (2), wave-wide HBM (3),
    parallel compact-layout (4) and batch HBM (5) kernels give the oracle's
    results on the same inputs."""
    rng = np.random.default_rng(77)
    dbs, K, prefill, req = 700, 300, 3000, 4
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(variant)
    try:
        for step in range(5):
            batch = _random_state_stream(rng, st, K, prefill)
            seq = np.full(req, prefill + 3)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == variant
            np.testing.assert_array_equal(g_miss, e_miss)
            np.testing.assert_array_equal(g_slots, e_slots)
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)


@pytest.mark.parametrize("dbs,K", [(64, 64), (64, 200), (37, 90), (1, 8)])
@pytest.mark.parametrize("variant", [0, 2, 3, 5])
def test_sieve_variants_agree_small_rows(kvops, variant, dbs, K):
    """Rows of at most 64 slots (the parallel kernel's register path when
    steps wrap the hand): the sequential LDS (0), parallel (2), wave-wide HBM
    (3) and batch HBM (5) kernels give the oracle's results, with repeats,
    conversions and hand wraps (topK above dbs wraps every step), invalid
    and decode-extension positions, and padding rows."""
    rng = np.random.default_rng(dbs * 1000 + K)
    prefill, req = 4 * dbs + 20, 9
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(variant)
    try:
        for step in range(6):
            batch = _random_state_stream(rng, st, K, prefill)
            seq = np.full(req, prefill + 3)
            nr = req if step % 3 else req - 2  # padding rows get the dummy outputs
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, nr, max_num_reqs=req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, nr, req, K)
            assert kvops.last_sieve_variant() == variant
            msg = "variant {} step {}".format(variant, step)
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=msg)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=msg)
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


def test_sieve_small_rows_flag_shared_between_kernels(kvops):
    """Rows of 64 slots under the kernels in turn: the flag and token
    fingerprint one kernel writes (the parallel kernel's register path and
    the batch HBM kernel) are what the next one trusts.  After a kernel that
    leaves the flag alone (0, 3) the tokens no longer match the fingerprint:
    the parallel kernel checks the row in full and flags it again, the batch
    kernel in its bitmap form (tokens below the table size, as here) takes
    the in-order recurrence, which clears it.  Full state against the oracle
    after every step."""
    rng = np.random.default_rng(4242)
    dbs, K, prefill, req = 64, 64, 300, 5
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    order = [2, 5, 2, 0, 2, 5, 3, 5, 2, 0, 5, 5, 2, 5]
    try:
        for step, variant in enumerate(order):
            kvops.sieve_force_variant(variant)
            batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.4)
            seq = np.full(req, prefill + 4)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == variant
            tag = "step {} variant {}".format(step, variant)
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=tag)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=tag)
            dev.assert_state_equal()
            flags = list(dev.hand.cpu().numpy()[0, :, 1])
            if variant == 2 or (variant == 5 and order[step - 1] in (2, 5)):
                assert flags == [CANON_FLAG] * req, tag
            elif variant == 5:  # after a kernel that leaves the flag alone
                assert flags == [0] * req, tag
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


def test_sieve_config3_parity(kvops):
    """Large-batch decode shapes (256 requests, topK 2048, 8192 slots, 10%
    misses; the parallel kernel's compact LDS layout): two steps, full state
    after each."""
    cfg = CONFIGS[3]
    st = orc.SieveState(1, cfg.req_num, cfg.dbs, cfg.top_k)
    for r in range(cfg.req_num):
        st.admit(r, cfg.prefill)
    dev = DevSieve(st)
    rng = np.random.default_rng(cfg.seed)
    req_pool = np.arange(cfg.req_num)
    seq = np.full(cfg.req_num, cfg.prefill)
    for step in range(2):
        batch = streams.state_batch(rng, st.tokens[0, :, :cfg.dbs], cfg.prefill, cfg.top_k, cfg.miss_ratio)
        e_slots, e_miss = st.update(0, batch, req_pool, seq, cfg.req_num)
        g_slots, g_miss, _ = dev.update(kvops, 0, batch, req_pool, seq, cfg.req_num, cfg.req_num, cfg.top_k)
        assert kvops.last_sieve_variant() == 4
        np.testing.assert_array_equal(g_miss, e_miss)
        np.testing.assert_array_equal(g_slots, e_slots)
        dev.assert_state_equal()
    assert kvops.read_overflow() == 0


def test_sieve_config4_parity(kvops):
    """The slot-limit stress shapes (4 requests, 65518 slots, topK 8192, a
    262144-entry table kept in HBM) with 90% misses drawn from the keys whose
    Knuth hashes share the table's first 40,960 homes: over 7,000 evictions per
    request on every step inside one long probe run, full state after each."""
    cfg = CONFIGS[4]
    st = orc.SieveState(1, cfg.req_num, cfg.dbs, cfg.top_k)
    for r in range(cfg.req_num):
        st.admit(r, cfg.prefill)
    dev = DevSieve(st)
    rng = np.random.default_rng(cfg.seed)
    pool = streams.adversarial_pool(cfg.prefill, cfg.adversarial_hash_below)
    req_pool = np.arange(cfg.req_num)
    seq = np.full(cfg.req_num, cfg.prefill)
    for step in range(4):
        batch = streams.state_batch(rng, st.tokens[0, :, :cfg.dbs], cfg.prefill, cfg.top_k, cfg.miss_ratio,
                                    miss_pool=pool)
        e_slots, e_miss = st.update(0, batch, req_pool, seq, cfg.req_num, threads=4)
        print("c4 step", step, "misses per request", e_miss.sum(axis=1), flush=True)
        assert e_miss.sum(axis=1).min() >= 7000
        g_slots, g_miss, _ = dev.update(kvops, 0, batch, req_pool, seq, cfg.req_num, cfg.req_num, cfg.top_k)
        assert kvops.last_sieve_variant() == 5
        np.testing.assert_array_equal(g_miss, e_miss)
        np.testing.assert_array_equal(g_slots, e_slots)
        dev.assert_state_equal()
    assert kvops.read_overflow() == 0


def test_sieve_wrap_fallback_large_table(kvops):
    """More misses than slots (the hand wraps within a step) on a table above
    4096 cells: the parallel kernel hands the row to the in-order recurrence
    run by a whole wave."""
    rng = np.random.default_rng(31)
    dbs, K, prefill, req = 600, 1800, 20000, 3
    st = orc.SieveState(1, req, dbs, K)
    assert st.ht_size > 4096
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    for step in range(3):
        batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.7)
        seq = np.full(req, prefill + 2)
        e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
        g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
        assert kvops.last_sieve_variant() == 2
        np.testing.assert_array_equal(g_miss, e_miss)
        np.testing.assert_array_equal(g_slots, e_slots)
        dev.assert_state_equal()
    assert kvops.read_overflow() == 0


def test_sieve_sequential_lds_wave_path(kvops):
    """The sequential LDS kernel on a table above 4096 cells (one wave per
    probe, sweep and shift step): large-batch decode shapes, one step."""
    cfg = CONFIGS[3]
    req = 32
    st = orc.SieveState(1, req, cfg.dbs, cfg.top_k)
    assert st.ht_size > 4096
    for r in range(req):
        st.admit(r, cfg.prefill)
    dev = DevSieve(st)
    rng = np.random.default_rng(5)
    kvops.sieve_force_variant(0)
    try:
        for step in range(2):
            batch = streams.state_batch(rng, st.tokens[0, :, :cfg.dbs], cfg.prefill, cfg.top_k, 0.3)
            e_slots, e_miss = st.update(0, batch, np.arange(req), np.full(req, cfg.prefill), req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), np.full(req, cfg.prefill), req, req,
                                            cfg.top_k)
            assert kvops.last_sieve_variant() == 0
            np.testing.assert_array_equal(g_miss, e_miss)
            np.testing.assert_array_equal(g_slots, e_slots)
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)


@pytest.mark.parametrize("dbs,K,prefill", [(64, 64, 256), (37, 100, 300), (16, 48, 12), (64, 200, 90)])
def test_sieve_small_rows_inorder_paths(kvops, dbs, K, prefill):
    """Rows of up to 64 slots whose steps wrap the hand: after a wrap the row
    takes the in-order decisions in registers and the parallel table update,
    retrying the parallel form after 8 and 16 wrapping steps; a row whose
    consistency flag was cleared takes the one-lane recurrence.  Full state after every step
    (partial visited bytes, empty slots, duplicates, invalid positions)."""
    rng = np.random.default_rng(dbs * 1000 + K)
    req = 4
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    for step in range(24):
        if step == 12:
            dev.hand[0, 1, 1] = 0  # row 1 no longer known consistent: checked again, one-lane path meanwhile
        if step == 14:
            # row 2's tokens edited outside the kernel (a duplicated token), the flag cleared as
            # the interface asks: the row is checked again and takes the exact one-lane recurrence
            live = np.nonzero(st.tokens[0, 2, :dbs] >= 0)[0]
            if len(live) >= 2:
                a_, b_ = int(live[0]), int(live[1])
                st.tokens[0, 2, a_] = st.tokens[0, 2, b_]
                dev.tokens[0, 2, a_] = int(st.tokens[0, 2, b_])
                dev.hand[0, 2, 1] = 0
        if step == 16:
            # row 3: one more live token than table entries with the flag still set; the count
            # check catches it
            empty = np.nonzero(st.tokens[0, 3, :dbs] < 0)[0]
            if len(empty):
                st.tokens[0, 3, int(empty[0])] = prefill - 1
                dev.tokens[0, 3, int(empty[0])] = prefill - 1
        batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.8)
        seq = np.full(req, prefill + 2)
        e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
        g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
        np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
        np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
        dev.assert_state_equal()
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("variant", [5, 3])
def test_sieve_hbm_noncanonical_table(kvops, variant):
    """A table that is not canonical (two entries swapped so that probe
    paths break, and an entry naming an empty slot): the batch kernel takes
    its in-order path, and both HBM kernels give what the oracle gives on the
    same table (the reference's probe semantics, whatever the table holds)."""
    rng = np.random.default_rng(19)
    dbs, K, prefill, req = 900, 256, 4000, 3
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    # row 0: swap two occupied cells of one cluster; row 1: an entry naming an
    # empty slot; row 2 stays canonical
    occ = np.nonzero(st.ht[0, 0])[0]
    a, b = int(occ[10]), int(occ[11])
    st.ht[0, 0, a], st.ht[0, 0, b] = st.ht[0, 0, b], st.ht[0, 0, a]
    st.tokens[0, 1, 5] = -1
    dev = DevSieve(st)
    kvops.sieve_force_variant(variant)
    try:
        for step in range(3):
            batch = _random_state_stream(rng, st, K, prefill)
            seq = np.full(req, prefill)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == variant
            np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
            np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("form", [5, 6])  # table changes: parallel rebuild, or in the batch kernel
def test_sieve_batch_kernel_wraps_and_dups(kvops, form, seed):
    """The batch HBM kernel on rows whose steps sometimes wrap the hand
    (more misses than slots: the in-order path) and sometimes do not,
    with duplicate positions, invalid and decode-extension positions."""
    rng = np.random.default_rng(900 + seed)
    dbs = int(rng.integers(60, 400))
    K = int(rng.integers(50, 600))
    prefill = int(rng.integers(dbs + 10, 6 * dbs))
    req = 4
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(form)
    try:
        for step in range(6):
            seq = np.full(req, prefill + 5)
            hi = prefill + 9 if step % 2 else dbs + 50
            batch = rng.integers(-2, hi, size=(req, K)).astype(np.int32)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == 5
            np.testing.assert_array_equal(g_miss, e_miss, err_msg="seed {} step {}".format(seed, step))
            np.testing.assert_array_equal(g_slots, e_slots, err_msg="seed {} step {}".format(seed, step))
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


CANON_FLAG = 0x4B565843  # sieve_hand[row][1] of a row a SIEVE kernel left consistent


@pytest.mark.parametrize("variant,prefill,dbs", [(2, 1500, 700), (4, 1500, 700), (5, 1500, 700), (5, 5000, 700),
                                                 (6, 1500, 700), (2, 400, 64)])
def test_sieve_flag_with_token_edited_in_place(kvops, variant, prefill, dbs):
    """sieve_hand[row][3] carries a fingerprint of the tokens a kernel left
    with the consistency flag.  A caller that changes a token value in place
    and leaves element 1 set (the reference's results depend only on tokens,
    visited bits, table and hand: hisp_sieve_update.cpp:103-111) gets the
    reference's results: the fingerprint no longer matches, so the row is
    checked in full (or runs the in-order recurrence) instead of being trusted.
    Variants: 2 the parallel LDS kernel (direct token map), 4 its compact
    form, 5 the batch HBM kernel (token bitmap below the table size, 2048
    cells, or a token map above it), 6 the batch kernel without the rebuild;
    with 64 slots the parallel kernel's register path."""
    rng = np.random.default_rng(31 + variant)
    K, req = 200, 3
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(variant)
    try:
        for step in range(5):
            batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.3)
            if step == 2:
                # row 1: a resident token becomes one the row does not hold
                assert int(dev.hand[0, 1, 1]) == CANON_FLAG
                toks = st.tokens[0, 1, :dbs]
                s = int(np.nonzero(toks >= 0)[0][5])
                t_old = int(toks[s])
                absent = np.setdiff1d(np.arange(prefill), toks)
                t_new = int(absent[rng.integers(len(absent))])
                st.tokens[0, 1, s] = t_new
                dev.tokens[0, 1, s] = t_new
                batch[1, [0, 9, 77]] = t_new
                batch[1, [3, 40]] = t_old
            seq = np.full(req, prefill + 4)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == (5 if variant == 6 else variant)
            msg = "variant {} prefill {} dbs {} step {}".format(variant, prefill, dbs, step)
            if step == 2:
                # the table has no entry for the new value: the reference misses it
                assert e_miss[1, 0] == 1, msg
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=msg)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=msg)
            dev.assert_state_equal()
            flags = dev.hand.cpu().numpy()[0, :, 1]
            if step == 1:
                assert list(flags) == [CANON_FLAG] * req, msg
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("prefill", [40000, 12000])  # tokens past the table size (a token map), or below it
@pytest.mark.parametrize("form", [5, 6])  # table changes: parallel rebuild, or in the batch kernel
def test_sieve_batch_second_pass(kvops, form, prefill):
    """Steps whose hand turns the whole ring (every slot visited) and then
    evicts slots it passed earlier in the step: tokens hit before the turn are
    evicted after it, so their next occurrences miss and the ones after those
    hit the new slots.  With topK < dbs the batch kernel decides such a step
    in its one pass (the row's consistency flag is set after every step; the
    in-order recurrence clears it), equal to the oracle."""
    dbs, K, req = 3000, 2048, 3
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
        st.hand[0, r, 0] = dbs - 100 + 10 * r  # the turn also crosses the ring's end
    bits = np.zeros(st.vis_stride * 8, dtype=bool)
    bits[:dbs] = True
    all_visited = np.packbits(bits, bitorder="little")
    rng = np.random.default_rng(77)
    dev = DevSieve(st)
    kvops.sieve_force_variant(form)
    try:
        for step in range(4):
            st.vis[0, :, :] = all_visited
            dev.vis.copy_(to_dev(st.vis))
            batch = np.empty((req, K), dtype=np.int32)
            for r in range(req):
                h0 = int(st.hand[0, r, 0])
                early = st.tokens[0, r, (h0 + np.arange(64)) % dbs].copy()
                fresh = rng.choice(np.setdiff1d(np.arange(prefill), st.tokens[0, r, :dbs]), size=1200, replace=False)
                rest = rng.integers(-2, prefill + 9, size=K - 64 - 1200 - 128)
                batch[r] = np.concatenate([early, fresh, early, early[::-1], rest])
            seq = np.full(req, prefill + 5)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == 5
            msg = "form {} prefill {} step {}".format(form, prefill, step)
            # the scenario: hits, then the same tokens evicted (misses), then hits again
            assert not e_miss[:, :64].any() and e_miss[:, 1264:1328].all() and not e_miss[:, 1328:1392].any(), msg
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=msg)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=msg)
            dev.assert_state_equal()
            assert (dev.hand.cpu().numpy()[0, :, 1] == CANON_FLAG).all(), msg
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("prefill", [5000, 1500])
def test_sieve_batch_consistency_flag(kvops, prefill):
    """The batch HBM kernel sets a row's consistency flag when it leaves the
    row consistent, and then counts the row's live tokens and entries instead
    of checking its table (with tokens below the table size, 2048 cells here,
    the step's tokens go in a bitmap instead of a token map).  A row edited
    outside the kernel with the flag
    cleared (an entry moved past an empty cell) is checked in full and takes
    the in-order path, which clears the flag; a row left with one more live
    token than entries with the flag set is caught by the counts.  Full state
    against the oracle after every step."""
    rng = np.random.default_rng(77)
    dbs, K, req = 700, 200, 3
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    H = st.ht.shape[-1]
    kvops.sieve_force_variant(5)
    try:
        for step in range(8):
            if step == 3:
                # row 1: the entry of an occupied cell moved to an empty cell
                # past the end of its cluster (an empty cell between its home
                # and its new cell), the flag cleared as the interface asks
                ht = st.ht[0, 1]
                c = int(np.nonzero(ht)[0][0])
                x = c
                while ht[x] != 0:
                    x = (x + 1) % H
                y = (x + 1) % H
                while ht[y] != 0:
                    y = (y + 1) % H
                ht[y], ht[c] = ht[c], 0
                dev.ht[0, 1, y] = int(ht[y])
                dev.ht[0, 1, c] = 0
                dev.hand[0, 1, 1] = 0
            if step == 5:
                # row 2: the entry at the end of a cluster removed (a live
                # token without an entry), the flag left set
                ht = st.ht[0, 2]
                c = int(np.nonzero((ht != 0) & (np.roll(ht, -1) == 0))[0][0])
                ht[c] = 0
                dev.ht[0, 2, c] = 0
            batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.3)
            seq = np.full(req, prefill + 4)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == 5
            np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
            np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
            dev.assert_state_equal()
            flags = dev.hand.cpu().numpy()[0, :, 1]
            if step == 0:
                assert list(flags) == [CANON_FLAG] * req
            if step == 3:
                assert flags[1] == 0 and flags[0] == CANON_FLAG and flags[2] == CANON_FLAG
            if step == 5:
                assert flags[2] == 0 and flags[0] == CANON_FLAG
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("variant", [-1, 5])
def test_stale_flag_after_table_rebuild(kvops, variant):
    """A row re-seeded outside the admission path: new tokens with one token
    in two slots, the table rebuilt by sieve_ht_init (which keeps the first
    of the two), the hand record left as it was, its consistency flag still
    set.  The live-token count exceeds the table's entries, so the kernels
    (the LDS kernel at this shape, and the batch HBM kernel) check the row
    and take the in-order path; the results match the oracle on the same
    row."""
    import torch
    rng = np.random.default_rng(31)
    dbs, K, prefill, req = 300, 128, 2000, 3
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(variant)
    try:
        for step in range(6):
            if step == 3:
                assert int(dev.hand[0, 1, 1]) == CANON_FLAG
                tok = rng.choice(prefill, size=dbs, replace=False).astype(np.int32)
                tok[7] = tok[3]
                st.tokens[0, 1, :dbs] = tok
                orc.sieve_ht_init(st.tokens, st.ht, 1, 1, 1, req, dbs, st.padded, st.ht_size)
                dev.tokens[0, 1, :dbs] = torch.from_numpy(tok).cuda()
                kvops.sieve_ht_init(dev.tokens.data_ptr(), dev.ht.data_ptr(), dev.prefill.data_ptr(), 1, 1, 1,
                                    req, dbs, st.padded, st.ht_size, 0, 1)
                torch.cuda.synchronize()
                dev.assert_state_equal()
                assert int(dev.hand[0, 1, 1]) == CANON_FLAG  # the rebuild cannot clear it
            batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.3)
            seq = np.full(req, prefill + 4)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            if variant >= 0:
                assert kvops.last_sieve_variant() == variant
            np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
            np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


def test_consistency_flag_shared_between_kernels(kvops):
    """Every variant on the same rows in turn: the flag one kernel sets (the
    LDS kernels and the batch HBM kernel) is what the next one trusts, and
    the kernels that leave it alone keep the row consistent.  Full state
    against the oracle after every step; the flag is set after the steps of
    the kernels that set it."""
    rng = np.random.default_rng(41)
    dbs, K, prefill, req = 300, 128, 1500, 3
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    order = [2, 5, 3, 5, 4, 5, 0, 5, 1, 5, 2, 2, 5, 5]
    try:
        for step, variant in enumerate(order):
            kvops.sieve_force_variant(variant)
            batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.3)
            seq = np.full(req, prefill + 4)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == variant
            tag = "step {} variant {}".format(step, variant)
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=tag)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=tag)
            dev.assert_state_equal()
            if variant in (2, 4, 5):
                assert list(dev.hand.cpu().numpy()[0, :, 1]) == [CANON_FLAG] * req, tag
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("prefill", [262149, 400000])
def test_sieve_batch_tokens_beyond_map(kvops, prefill):
    """The batch HBM kernel with prefill lengths past its token map (2^18
    tokens) and past the table size: steps whose tokens all fit take the
    batch path, a row holding or asked for a larger token takes the
    in-order path.  Full state against the oracle after every step."""
    rng = np.random.default_rng(prefill)
    dbs, K, req = 300, 128, 3
    st = orc.SieveState(1, req, dbs, K)
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(5)
    try:
        for step in range(8):
            if step < 3:
                # misses from below the map's reach first, then from the whole prefill
                batch = _random_state_stream(rng, st, K, 200000, miss_frac=0.3)
            else:
                batch = _random_state_stream(rng, st, K, prefill, miss_frac=0.3)
            seq = np.full(req, prefill + 4)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == 5
            np.testing.assert_array_equal(g_miss, e_miss, err_msg="step {}".format(step))
            np.testing.assert_array_equal(g_slots, e_slots, err_msg="step {}".format(step))
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("form", [5, 6])  # table changes: parallel rebuild, or in the batch kernel
def test_sieve_batch_fuzz_flagged(kvops, form, seed):
    """The batch HBM kernel over random shapes whose tokens lie below the
    table size (so flagged rows take the token bitmap), with the flag of a
    random row cleared now and then, mixed hit/miss streams with duplicates
    and invalid positions: full state against the oracle after every step."""
    rng = np.random.default_rng(7000 + seed)
    dbs = int(rng.integers(60, 1500))
    K = int(rng.integers(50, 900))
    req = int(rng.integers(1, 6))
    st = orc.SieveState(1, req, dbs, K)
    prefill = int(rng.integers(dbs + 10, st.ht_size + 1))
    for r in range(req):
        st.admit(r, prefill)
    dev = DevSieve(st)
    kvops.sieve_force_variant(form)
    try:
        for step in range(8):
            if step > 0 and rng.random() < 0.4:
                dev.hand[0, int(rng.integers(0, req)), 1] = 0
            batch = _random_state_stream(rng, st, K, prefill, miss_frac=float(rng.random() * 0.6))
            seq = np.full(req, prefill + 4)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == 5
            tag = "seed {} dbs {} K {} prefill {} step {}".format(seed, dbs, K, prefill, step)
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=tag)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=tag)
            dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("misses", [1, 3, 40, 400])
@pytest.mark.parametrize("form", [5, 6])  # table changes: parallel rebuild, or in the batch kernel
def test_sieve_batch_cluster_walks(kvops, form, misses):
    """The batch HBM kernel's deletion walk over one long cluster: every
    token's home lies in the first eighth of the table, so the entries pile
    up and each deletion's hole is carried through the cluster.  Steps with
    1 to 400 misses per row exercise the windows decided in parallel (one
    hole), the holes taken in order (several), the lanes packed and the
    spill to the hole bitmap (more than 64).  Full state against the oracle
    after every step."""
    import torch
    rng = np.random.default_rng(900 + misses)
    dbs, K, req = 3000, 512, 2
    st = orc.SieveState(1, req, dbs, K)
    H = st.ht_size
    prefill = 1 << 16
    t = np.arange(prefill, dtype=np.int64)
    home = (((t * 2654435761) & 0xFFFFFFFF) >> 16) & (H - 1)
    pool = t[home < H // 8].astype(np.int32)
    for r in range(req):
        st.admit(r, prefill)
        st.tokens[0, r, :dbs] = rng.choice(pool, size=dbs, replace=False)
    orc.sieve_ht_init(st.tokens, st.ht, 0, req, 1, req, dbs, st.padded, H)
    dev = DevSieve(st)
    kvops.sieve_force_variant(form)
    try:
        for step in range(6):
            batch = np.empty((req, K), dtype=np.int32)
            for r in range(req):
                live = st.tokens[0, r, :dbs]
                hits = rng.choice(live, size=K - misses)
                fresh = np.setdiff1d(pool, live)
                batch[r] = rng.permutation(np.concatenate([hits, rng.choice(fresh, size=misses, replace=False)]))
            seq = np.full(req, prefill)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == 5
            tag = "misses {} step {}".format(misses, step)
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=tag)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=tag)
            dev.assert_state_equal()
            assert list(dev.hand.cpu().numpy()[0, :, 1]) == [CANON_FLAG] * req, tag
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("form", [5, 6])  # table changes: parallel rebuild, or in the batch kernel
def test_sieve_batch_scratch_across_shapes(kvops, form):
    """The batch HBM kernel's per-row scratch is laid out by table size and
    shared by every launch on the stream: launches on one shape, then on a
    larger one with more rows, then the first again, all match the oracle
    (each launch leaves the scratch zeroed)."""
    shapes = [(7, 40, 64, 300), (4, 3000, 1000, 20000), (7, 40, 64, 300)]
    rng = np.random.default_rng(4)
    kvops.sieve_force_variant(form)
    try:
        for i, (req, dbs, K, prefill) in enumerate(shapes):
            st = orc.SieveState(1, req, dbs, K)
            for r in range(req):
                st.admit(r, prefill)
            dev = DevSieve(st)
            for step in range(3):
                batch = _random_state_stream(rng, st, K, prefill)
                seq = np.full(req, prefill + 4)
                e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
                g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
                assert kvops.last_sieve_variant() == 5
                np.testing.assert_array_equal(g_miss, e_miss, err_msg="shape {} step {}".format(i, step))
                np.testing.assert_array_equal(g_slots, e_slots, err_msg="shape {} step {}".format(i, step))
                dev.assert_state_equal()
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0


@pytest.mark.parametrize("case", ["wrap", "past-2^16"])
def test_sieve_table_rebuild_cluster_edges(kvops, case):
    """The parallel table rebuild where the cell order matters most: "wrap"
    puts every token's home in the last eighth of an 8192-cell table, so the
    clusters run past the table's end into cell 0; "past-2^16" (a 131072-cell
    table) homes the tokens in the 16384 cells below 65536, so the clusters run
    past cell 65535 and the order must start after it.  Steps with 1 to 300
    misses per row, full state against the oracle after every step."""
    rng = np.random.default_rng(31 if case == "wrap" else 32)
    dbs, K, req = (3000, 512, 2) if case == "wrap" else (40000, 4096, 1)
    st = orc.SieveState(1, req, dbs, K)
    H = st.ht_size
    assert H == (8192 if case == "wrap" else 131072)
    prefill = 1 << 18
    t = np.arange(prefill, dtype=np.int64)
    home = (((t * 2654435761) & 0xFFFFFFFF) >> 16) & (H - 1)
    lo = H - H // 8 if case == "wrap" else 65536 - 16384
    pool = t[(home >= lo) & (home < lo + (H // 8 if case == "wrap" else 16384))].astype(np.int32)
    assert len(pool) > dbs + 4 * 300
    for r in range(req):
        st.admit(r, prefill)
        st.tokens[0, r, :dbs] = rng.choice(pool, size=dbs, replace=False)
    orc.sieve_ht_init(st.tokens, st.ht, 0, req, 1, req, dbs, st.padded, H)
    dev = DevSieve(st)
    kvops.sieve_force_variant(5)
    try:
        for step, misses in enumerate([1, 40, 300, 7]):
            batch = np.empty((req, K), dtype=np.int32)
            for r in range(req):
                live = st.tokens[0, r, :dbs]
                hits = rng.choice(live, size=K - misses)
                fresh = np.setdiff1d(pool, live)
                batch[r] = rng.permutation(np.concatenate([hits, rng.choice(fresh, size=misses, replace=False)]))
            seq = np.full(req, prefill)
            e_slots, e_miss = st.update(0, batch, np.arange(req), seq, req)
            g_slots, g_miss, _ = dev.update(kvops, 0, batch, np.arange(req), seq, req, req, K)
            assert kvops.last_sieve_variant() == 5
            tag = "{} step {}".format(case, step)
            np.testing.assert_array_equal(g_miss, e_miss, err_msg=tag)
            np.testing.assert_array_equal(g_slots, e_slots, err_msg=tag)
            dev.assert_state_equal()
            assert list(dev.hand.cpu().numpy()[0, :, 1]) == [CANON_FLAG] * req, tag
    finally:
        kvops.sieve_force_variant(-1)
    assert kvops.read_overflow() == 0
