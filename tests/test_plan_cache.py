"""PlanCache's contract (J/tornado/PlanCache.java:25-161) on fake plans (CPU only): LRU order,
the plan-count and byte budgets, retry-once after a failed first use, close()."""
import pytest

from jitcast_amd.plans import PlanCache


class FakePlan:
    def __init__(self, key, nbytes, log):
        self.key, self.nbytes, self.log, self.closed = key, nbytes, log, False

    def device_bytes(self):
        return self.nbytes

    def close(self):
        self.closed = True
        self.log.append(("close", self.key))


def test_lru_within_count_and_bytes():
    log = []
    c = PlanCache(max_plans=2, max_bytes=100)
    build = lambda k: FakePlan(k, 40, log)  # noqa: E731
    for k in ("a", "b"):
        assert c.run(k, build, lambda p: p.key) == k
    c.run("a", build, lambda p: None)  # touches a: b is now the eldest
    c.run("c", build, lambda p: None)  # count budget evicts b
    assert c.keys() == ["a", "c"] and ("close", "b") in log
    assert c.cached_bytes() == 80
    big = lambda k: FakePlan(k, 70, log)  # noqa: E731
    c.run("d", big, lambda p: None)  # count evicts a, then bytes evict c (70 + 40 > 100)
    assert c.keys() == ["d"] and c.cached_bytes() == 70


def test_cached_plan_is_reused_not_rebuilt():
    log, built = [], []
    c = PlanCache(4, 1000)

    def build(k):
        built.append(k)
        return FakePlan(k, 1, log)

    for _ in range(3):
        c.run("x", build, lambda p: None)
    assert built == ["x"]


def test_failed_first_use_is_closed_and_not_cached_when_alone():
    log = []
    c = PlanCache(4, 1000)

    def use(p):
        raise RuntimeError("out of memory")

    with pytest.raises(RuntimeError, match="out of memory"):
        c.run("x", lambda k: FakePlan(k, 1, log), use)
    assert c.keys() == [] and log == [("close", "x")]


def test_failed_first_use_clears_cache_and_retries_once():
    log, attempts = [], []
    c = PlanCache(4, 1000)
    c.run("a", lambda k: FakePlan(k, 1, log), lambda p: None)

    def use(p):
        attempts.append(p.key)
        if len(attempts) == 1:
            raise RuntimeError("transient")
        return "ok"

    assert c.run("b", lambda k: FakePlan(k, 1, log), use) == "ok"
    assert attempts == ["b", "b"]
    assert ("close", "a") in log  # the other plans were cleared before the retry
    assert c.keys() == ["b"]


def test_second_failure_propagates_with_the_first_attached():
    log = []
    c = PlanCache(4, 1000)
    c.run("a", lambda k: FakePlan(k, 1, log), lambda p: None)

    def use(p):
        raise RuntimeError(f"fail {len(log)}")

    with pytest.raises(RuntimeError) as ei:
        c.run("b", lambda k: FakePlan(k, 1, log), use)
    assert isinstance(ei.value.__context__, RuntimeError)
    assert c.keys() == []


def test_rejects_empty_budgets_and_close_closes_all():
    with pytest.raises(ValueError):
        PlanCache(0, 1)
    log = []
    c = PlanCache(3, 100)
    for k in "abc":
        c.run(k, lambda key: FakePlan(key, 1, log), lambda p: None)
    c.close()
    assert sorted(x[1] for x in log) == ["a", "b", "c"] and c.keys() == []
