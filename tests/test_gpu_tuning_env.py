"""The kernel-choice switches a context takes from the environment when it is made (WE_GEMM_CFG, WE_GEMM_PATH,
WE_GEMM_SPLITK, WE_GEMM_REDUCE_XCD, WE_ATTN_PATH, WE_INT4_PATH; include/we.h, we_set_tuning). Each case makes a
context of its own with one variable set and reads every switch back through we_set_tuning, which returns the
previous value. Unknown values keep the defaults. Additive: the reference picks kernel variants in its tuner
(src/bench/tune.ts:5-30), not through the environment."""
import os

import pytest

import we

pytestmark = pytest.mark.gpu

DEFAULTS = {"gemm_cfg": -1, "gemm_generic": 0, "gemm_splitk": -1, "gemm_reduce_xcd": 1, "attn_path": 0,
            "int4_path": 0}
ENV_OF = {"gemm_cfg": "WE_GEMM_CFG", "gemm_generic": "WE_GEMM_PATH", "gemm_splitk": "WE_GEMM_SPLITK",
          "gemm_reduce_xcd": "WE_GEMM_REDUCE_XCD", "attn_path": "WE_ATTN_PATH", "int4_path": "WE_INT4_PATH"}


def switches_of_new_context(env):
    old = {k: os.environ.get(k) for k in ENV_OF.values()}
    try:
        for k in ENV_OF.values():
            os.environ.pop(k, None)
        os.environ.update(env)
        g = we.Graph(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    try:
        got = {}
        for key in DEFAULTS:
            got[key] = g.set_tuning(key, DEFAULTS[key])
        return got
    finally:
        g.destroy()


@pytest.mark.parametrize("key,value,want", [
    ("attn_path", "registers", 1), ("attn_path", "ring", 2), ("attn_path", "mfma16", 3), ("attn_path", "other", 0),
    ("int4_path", "generic", 1), ("int4_path", "shared", 2), ("int4_path", "pipe", 3), ("int4_path", "other", 0),
    ("gemm_cfg", "5", 5), ("gemm_generic", "generic", 1), ("gemm_splitk", "off", 0), ("gemm_splitk", "6", 6),
    ("gemm_splitk", "x", -1), ("gemm_reduce_xcd", "off", 0)])
def test_environment_sets_one_switch(key, value, want):
    got = switches_of_new_context({ENV_OF[key]: value})
    assert got == {**DEFAULTS, key: want}


def test_no_environment_gives_the_defaults():
    assert switches_of_new_context({}) == DEFAULTS


def test_a_context_keeps_its_switches_when_the_environment_changes(graph):
    """Launches read the context, never the environment: setting a variable after the context exists changes
    nothing in it."""
    before = graph.set_tuning("attn_path", 0)
    os.environ["WE_ATTN_PATH"] = "ring"
    try:
        assert graph.set_tuning("attn_path", before) == 0
    finally:
        os.environ.pop("WE_ATTN_PATH", None)
