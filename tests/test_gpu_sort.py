"""The radix sort and the count scan called directly through the C ABI (include/b2c_kernels.h), against
numpy's stable argsort and cumsum on seeded keys: every tile size of the sort (2048-, 4096- and 8192-key
tiles) and digit width (8 and 9 bits),
partial bit ranges, a device-side live count, heavy digit skew (the culled 0xFFFFFFFF depth keys) and one
or two value arrays, including the "no values: sort the positions" form the tile pass uses
(src/gpu/binning.cu:116-118,140-142 sort with cub::DeviceRadixSort::SortPairs, which is stable)."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from b2ctrain_amd import _native


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _sort(keys, vals, vals2, begin, end, live=None):
    """Run b2c_hip_radix_sort_kv2; returns (keys_out, vals_out, vals2_out) as numpy (live entries only)."""
    L = _native.lib()
    n = keys.size
    kd, vd = _dev(keys), None if vals is None else _dev(vals)
    v2d = None if vals2 is None else _dev(vals2)
    out = [torch.empty(n, dtype=torch.int32, device="cuda") for _ in range(6)]
    v2o = [torch.empty(n, dtype=torch.int32, device="cuda") for _ in range(2)] if vals2 is not None else [None, None]
    tb = L.b2c_radix_sort_temp_bytes(n)
    tmp = torch.empty(tb, dtype=torch.uint8, device="cuda")
    n_dev = None if live is None else _dev(np.array([live], np.uint32))
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.b2c_hip_radix_sort_kv2(_p(kd), _p(vd), _p(v2d), _p(out[0]), _p(out[1]), _p(v2o[0]), _p(out[2]),
                                  _p(out[3]), _p(v2o[1]), C.c_uint32(n), _p(n_dev), C.c_int(begin), C.c_int(end),
                                  _p(tmp), C.c_size_t(tb), stream)
    _native.check(rc, "radix sort")
    torch.cuda.synchronize()
    m = n if live is None else live
    ko = out[0].cpu().numpy().view(np.uint32)[:m]
    vo = out[1].cpu().numpy().view(np.uint32)[:m]
    v2 = None if vals2 is None else v2o[0].cpu().numpy().view(np.uint32)[:m]
    return ko, vo, v2


def _expect(keys, vals, vals2, begin, end, live=None):
    m = keys.size if live is None else live
    k = keys[:m]
    digits = (k >> np.uint32(begin)) & np.uint32((1 << (end - begin)) - 1) if end - begin < 32 else k
    perm = np.argsort(digits, kind="stable")
    v = np.arange(m, dtype=np.uint32) if vals is None else vals[:m]
    return k[perm], v[perm], None if vals2 is None else vals2[:m][perm]


CASES = [  # (n, key generator, begin, end)
    (1, "rand32", 0, 32),
    (777, "rand32", 0, 32),
    (4096, "dup", 0, 32),
    (4097, "dup", 0, 32),
    (300_001, "rand32", 0, 32),
    (1_000_000, "depth", 0, 32),
    (5_000_003, "tile15", 0, 15),
    (9_700_000, "tile15", 0, 15),
    (200_000, "rand32", 8, 20),
    # large sorts whose width is just over a multiple of 8 bits take 9-bit digits: one 9-bit pass for 9
    # bits, 9 + 8 for 17 (4K tile keys), 9 + 9 + 8 for 26 (from bit 3)
    (4_500_000, "tile17", 0, 17),
    (4_194_304, "rand32", 0, 9),
    (4_200_001, "rand32", 3, 29),
    # the ends of the 2048-key-tile range (2^22 keys and up take 4096-key tiles)
    (262_144, "dup", 0, 32),
    (4_194_303, "depth", 0, 32),
    (500_000, "rand32", 3, 29),
    (262_143, "depth", 0, 32),
]


def _keys(kind, n, rng):
    if kind == "rand32":
        return rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    if kind == "dup":
        return rng.integers(0, 37, n).astype(np.uint32) * np.uint32(0x01010101)
    if kind == "tile15":
        return rng.integers(0, 32400, n).astype(np.uint32)
    if kind == "tile17":  # 3840x2160: 129,600 tiles, and the sentinel key
        return rng.integers(0, 129_601, n).astype(np.uint32)
    if kind == "depth":  # view-z bits in [1, 10) and 40% culled splats at 0xFFFFFFFF
        z = rng.uniform(1.0, 10.0, n).astype(np.float32).view(np.uint32)
        return np.where(rng.random(n) < 0.4, np.uint32(0xFFFFFFFF), z).astype(np.uint32)
    raise ValueError(kind)


@pytest.mark.parametrize("n,kind,begin,end", CASES)
def test_radix_sort_matches_stable_argsort(n, kind, begin, end):
    rng = np.random.default_rng(n)
    keys = _keys(kind, n, rng)
    vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    print(f"sort n={n} kind={kind} bits=[{begin},{end})", flush=True)
    got = _sort(keys, vals, None, begin, end)
    exp = _expect(keys, vals, None, begin, end)
    assert np.array_equal(got[0], exp[0]) and np.array_equal(got[1], exp[1])


@pytest.mark.parametrize("n", [4099, 2_000_000, 6_000_001])
def test_radix_sort_two_values_positions(n):
    """The tile pass form: no input values (positions sorted) plus a second value array."""
    rng = np.random.default_rng(7 + n)
    keys = _keys("tile15", n, rng)
    vals2 = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    print(f"kv2 n={n}", flush=True)
    got = _sort(keys, None, vals2, 0, 15)
    exp = _expect(keys, None, vals2, 0, 15)
    for g, e in zip(got, exp):
        assert np.array_equal(g, e)


def test_radix_sort_two_values_32_bits():
    """Positions sorted and a second value array carried over four 8-bit passes."""
    n = 400_001
    rng = np.random.default_rng(11)
    keys = _keys("rand32", n, rng)
    vals2 = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    print(f"kv2 32 bits n={n}", flush=True)
    got = _sort(keys, None, vals2, 0, 32)
    exp = _expect(keys, None, vals2, 0, 32)
    for g, e in zip(got, exp):
        assert np.array_equal(g, e)


@pytest.mark.parametrize("n,live", [(6_000_000, 5_100_007), (36_000_000, 34_000_001)])
def test_radix_sort_two_values_positions_17_bits(n, live):
    """The 4K tile pass: 17-bit keys in a 9-bit and an 8-bit pass, positions and a second value array, a live
    count below the capacity (4096- and, from 2^25 keys, 8192-key tiles)."""
    rng = np.random.default_rng(17)
    keys = _keys("tile17", n, rng)
    vals2 = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    print(f"kv2 17 bits n={n} live={live}", flush=True)
    got = _sort(keys, None, vals2, 0, 17, live=live)
    exp = _expect(keys, None, vals2, 0, 17, live=live)
    for g, e in zip(got, exp):
        assert np.array_equal(g, e)


@pytest.mark.parametrize("cap,live", [(100_000, 70_001), (600_000, 410_001), (5_000_000, 4_100_000), (5_000, 0)])
def test_radix_sort_device_live_count(cap, live):
    rng = np.random.default_rng(cap)
    keys = _keys("rand32", cap, rng)
    vals = rng.integers(0, 2**32, cap, dtype=np.uint64).astype(np.uint32)
    print(f"live cap={cap} live={live}", flush=True)
    got = _sort(keys, vals, None, 0, 32, live=live)
    exp = _expect(keys, vals, None, 0, 32, live=live)
    assert np.array_equal(got[0], exp[0]) and np.array_equal(got[1], exp[1])


@pytest.mark.parametrize("n", [1, 1023, 1024, 1025, 1_000_000])
def test_count_scan_matches_cumsum(n):
    """b2c_hip_scan_counts: inclusive scan of tile_count gathered in depth order, total on the device."""
    L = _native.lib()
    rng = np.random.default_rng(n)
    counts = rng.integers(0, 50, n).astype(np.uint32)
    order = rng.permutation(n).astype(np.uint32)
    cd, od = _dev(counts), _dev(order)
    off = torch.empty(n, dtype=torch.int32, device="cuda")
    tot = torch.zeros(1, dtype=torch.int32, device="cuda")
    tb = L.b2c_scan_temp_bytes(n)
    tmp = torch.empty(tb, dtype=torch.uint8, device="cuda")
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"scan n={n}", flush=True)
    rc = L.b2c_hip_scan_counts(C.c_int(n), _p(od), _p(cd), _p(off), _p(tot), _p(tmp), C.c_size_t(tb), stream)
    _native.check(rc, "count scan")
    torch.cuda.synchronize()
    exp = np.cumsum(counts[order].astype(np.uint64)).astype(np.uint32)
    assert np.array_equal(off.cpu().numpy().view(np.uint32), exp)
    assert int(tot.cpu().numpy().view(np.uint32)[0]) == int(exp[-1])


def _ranges_expect(keys, n_tiles):
    """[first, last) of each tile in sorted keys, empty tiles [0, 0); tile_end = last, and tile_end[n_tiles] =
    the first sentinel key (>= n_tiles) or the key count (src/gpu/binning.cu:95-105 plus this build's copy)."""
    m = keys.size
    ranges = np.zeros((n_tiles, 2), np.uint32)
    tile_end = np.zeros(n_tiles + 1, np.uint32)
    for t in np.unique(keys[keys < n_tiles]):
        lo, hi = np.searchsorted(keys, t, "left"), np.searchsorted(keys, t, "right")
        ranges[t] = (lo, hi)
        tile_end[t] = hi
    tile_end[n_tiles] = np.searchsorted(keys, n_tiles, "left") if m else 0
    return ranges, tile_end


@pytest.mark.parametrize("case", ["dense", "gaps", "sentinels", "one", "empty", "all_sentinel", "live"])
def test_tile_ranges_write_every_tile(case):
    """b2c_hip_tile_ranges on outputs poisoned beforehand: every tile is written (the kernel clears the tiles
    no key names itself), including no keys at all, sentinel keys (>= n_tiles) and a device-side live count."""
    L = _native.lib()
    n_tiles = 5000
    rng = np.random.default_rng(len(case))
    live = None
    if case == "dense":
        keys = np.sort(rng.integers(0, n_tiles, 200_000)).astype(np.uint32)
    elif case == "gaps":
        keys = np.sort(rng.choice([3, 4, 900, 901, 2500, 4998], 3000)).astype(np.uint32)
    elif case == "sentinels":
        keys = np.sort(np.concatenate([rng.integers(10, 4000, 5000), np.full(77, n_tiles)])).astype(np.uint32)
    elif case == "one":
        keys = np.array([1234], np.uint32)
    elif case == "empty":
        keys = np.zeros(0, np.uint32)
    elif case == "all_sentinel":
        keys = np.full(10, n_tiles, np.uint32)
    else:  # launched for a capacity of 50,000 keys, 31,000 live (the binning's queued-before-the-count form)
        keys = np.sort(rng.integers(0, n_tiles, 50_000)).astype(np.uint32)
        live = 31_000
        keys[live:] = 0xFFFFFFFF  # past the live count: must not be read as keys
        keys[:live] = np.sort(keys[:live])
    m = keys.size
    kd = _dev(keys if m else np.zeros(1, np.uint32))
    ranges = _dev(np.full(n_tiles * 2, 0xDEADBEEF, np.uint32).view(np.int32))
    tile_end = _dev(np.full(n_tiles + 1, 0xDEADBEEF, np.uint32).view(np.int32))
    m_dev = None if live is None else _dev(np.array([live], np.uint32))
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"tile ranges case={case} m={m} live={live}", flush=True)
    rc = L.b2c_hip_tile_ranges(C.c_uint32(m), _p(m_dev), _p(kd), None, None, None, C.c_uint32(n_tiles), _p(ranges),
                               _p(tile_end), stream)
    _native.check(rc, "tile ranges")
    torch.cuda.synchronize()
    exp_r, exp_e = _ranges_expect(keys[: (m if live is None else live)], n_tiles)
    got_r = ranges.cpu().numpy().view(np.uint32).reshape(n_tiles, 2)
    got_e = tile_end.cpu().numpy().view(np.uint32)
    bad = np.flatnonzero((got_r != exp_r).any(1))
    assert bad.size == 0, f"ranges differ at tiles {bad[:10]}: {got_r[bad[:3]]} vs {exp_r[bad[:3]]}"
    assert np.array_equal(got_e, exp_e), f"tile_end differs at {np.flatnonzero(got_e != exp_e)[:10]}"
