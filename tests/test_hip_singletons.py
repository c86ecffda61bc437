"""The NumPy family's runtime singletons: a maker that takes another
singleton (the stager's and the pool's take the runtime) must not deadlock
when it is the first one created.  CPU-only: the makers are stand-ins."""

import threading

import pytest


@pytest.fixture
def hip():
    import importlib
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    return importlib.import_module("ozaki_jax_amd._hip")


def test_nested_singleton_creation_does_not_deadlock(hip):
    key_outer, key_inner = "_test_outer", "_test_inner"
    hip._state.pop(key_outer, None)
    hip._state.pop(key_inner, None)
    made = []

    def make_inner():
        made.append("inner")
        return object()

    def make_outer():
        inner = hip._get(key_inner, make_inner)  # nested, as _Stager(_rt())
        made.append("outer")
        return (inner,)

    out = []
    t = threading.Thread(target=lambda: out.append(hip._get(key_outer, make_outer)),
                         daemon=True)
    t.start()
    t.join(timeout=10)
    try:
        assert not t.is_alive(), "nested singleton creation deadlocked"
        assert made == ["inner", "outer"]
        assert out[0][0] is hip._state[key_inner]
    finally:
        hip._state.pop(key_outer, None)
        hip._state.pop(key_inner, None)
