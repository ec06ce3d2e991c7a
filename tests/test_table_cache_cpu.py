"""Host-side transfer-table cache policy (conversenet_amd.functional.TableCache, cacheable) and the
module's routing of unsupported geometries, on CPU tensors (no device needed)."""
import torch

from conversenet_amd import functional as Fh


def _key(w, b, geo=(1,), route=1):
    return Fh._cache_key("module", w, b, 1e-5, geo, route, torch.device("cpu"))


def test_in_place_update_replaces_entry_instead_of_adding():
    c = Fh.TableCache()
    w, b = torch.ones(1, 4, 3, 3), torch.zeros(1, 4, 1, 1)
    c.put(_key(w, b), torch.empty(100, dtype=torch.uint8), (w, b))
    assert c.get(_key(w, b)) is not None
    for _ in range(5):  # optimizer-style in-place steps
        w.mul_(0.5)
        assert c.get(_key(w, b)) is None
        c.put(_key(w, b), torch.empty(100, dtype=torch.uint8), (w, b))
    assert len(c.entries) == 1 and c.bytes == 100


def test_route_and_geometry_are_part_of_the_key():
    c = Fh.TableCache()
    w, b = torch.ones(1, 4, 3, 3), torch.zeros(1, 4, 1, 1)
    c.put(_key(w, b, route=1), torch.empty(10, dtype=torch.uint8), (w, b))
    assert c.get(_key(w, b, route=3)) is None
    assert c.get(_key(w, b, geo=(2,))) is None
    c.put(_key(w, b, route=3), torch.empty(20, dtype=torch.uint8), (w, b))
    assert len(c.entries) == 2 and c.bytes == 30


def test_lru_bounds():
    c = Fh.TableCache(max_entries=3, max_bytes=250)
    ts = [(torch.ones(1, 1, 1, 1), torch.zeros(1, 1, 1, 1)) for _ in range(5)]
    for w, b in ts:
        c.put(_key(w, b), torch.empty(100, dtype=torch.uint8), (w, b))
    assert len(c.entries) == 2 and c.bytes == 200
    assert c.get(_key(*ts[-1])) is not None and c.get(_key(*ts[0])) is None
    c.clear()
    assert c.bytes == 0 and not c.entries and not c.latest


def test_cacheable_rules():
    w = torch.nn.Parameter(torch.ones(1, 4, 3, 3))
    b = torch.nn.Parameter(torch.zeros(1, 4, 1, 1))
    assert not Fh.cacheable(w, b)  # autograd tracks them: training
    with torch.no_grad():
        assert Fh.cacheable(w, b)
    with torch.inference_mode():
        assert Fh.cacheable(w, b)  # parameters created outside inference mode keep a version counter
        k = torch.ones(1, 4, 3, 3)  # an activation made in inference mode (ConvReverseDataNet's psf)
        assert k.is_inference() and not Fh.cacheable(k, b)


def test_unsupported_geometries_are_routed_to_the_composition():
    w = torch.ones(1, 3, 3, 3) / 9
    assert Fh.supported(torch.empty(1, 3, 64, 64), w, 1, 1)
    assert not Fh.supported(torch.empty(1, 3, 5000, 8), w, 1, 1)
    assert not Fh.supported(torch.empty(1, 3, 8, 8), w, 5, 1, grad_weight=True)
    assert Fh.supported(torch.empty(1, 3, 8, 8), w, 5, 1, grad_x=True)
    assert Fh.supported(None, w, 1, 1, shape=(1, 3, 64, 64))


def test_concurrent_callers_keep_the_cache_consistent():
    """The op may be called from any host thread (the reference's cache is mutex-guarded,
    converse2d.cpp:56,70,90): eight threads hitting, filling and invalidating (in-place updates) one
    cache leave its byte count, entry bound and latest-version map consistent and raise nothing."""
    import random
    import threading

    c = Fh.TableCache(max_entries=16, max_bytes=1 << 30)
    params = [(torch.ones(1, 1, 1, 1), torch.zeros(1, 1, 1, 1)) for _ in range(40)]
    errors = []
    start = threading.Barrier(8)

    def worker(seed):
        rng = random.Random(seed)
        start.wait()
        try:
            for _ in range(3000):
                w, b = params[rng.randrange(len(params))]
                k = _key(w, b)
                if c.get(k) is None:
                    c.put(k, torch.empty(rng.choice((10, 20, 30)), dtype=torch.uint8), (w, b))
                if rng.random() < 0.05:
                    w.add_(0)  # an in-place update: bumps the version counter
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]
    assert len(c.entries) <= 16
    assert c.bytes == sum(t.numel() for t, _ in c.entries.values())
    assert all(c.latest[c._stem(k)] == k for k in c.entries)
