"""stablehlo.while on the CPU side: both text forms parse, captured values
become inputs of the while step, calls inside a region are inlined, and the
planner fixes the iteration count exactly when constants fix it (then the
runtime runs the body that many times with no host round trip)."""
import json

import pytest

from pjrtx_amd.hlo import Builder
from pjrtx_amd.pjrt import plugin


def _plan(text):
    return json.loads(plugin().plan_json(text))


def _counter_loop(start, bound, step, direction="LT", bound_in_state=False, start_param=False):
    b = Builder()
    x = b.param((4,), "f32")
    s0 = b.param((), "s32") if start_param else b.constant(start, "s32")
    bnd = b.constant(bound, "s32")
    state = [s0, x] + ([bnd] if bound_in_state else [])

    def cond(i, v, *rest):
        return b.compare(direction, i, rest[0] if bound_in_state else bnd)

    def body(i, v, *rest):
        return [b.add(i, b.constant(step, "s32")), b.multiply(v, v)] + list(rest)

    out = b.while_loop(state, cond, body)
    return b.build([out[1]])


@pytest.mark.parametrize("start,bound,step,direction,trips", [
    (0, 5, 1, "LT", 5),
    (0, 5, 1, "LE", 6),
    (3, 3, 1, "LT", 0),
    (0, 10, 3, "LT", 4),      # 0, 3, 6, 9
    (10, 0, -2, "GT", 5),     # 10, 8, 6, 4, 2
    (10, 0, -2, "GE", 6),
    (0, -3, 1, "LT", 0),
])
def test_static_trip_counts(start, bound, step, direction, trips):
    steps = _plan(_counter_loop(start, bound, step, direction))["steps"]
    assert [s["library"] for s in steps] == ["while"]
    assert steps[0]["while_trips"] == trips


def test_bound_passed_through_the_state_is_still_constant():
    steps = _plan(_counter_loop(0, 7, 1, bound_in_state=True))["steps"]
    assert steps[0]["while_trips"] == 7


def test_counts_that_depend_on_arguments_are_not_fixed():
    assert _plan(_counter_loop(0, 7, 1, start_param=True))["steps"][0]["while_trips"] == -1
    # an increasing counter tested with GT never runs or never stops: not fixed
    assert _plan(_counter_loop(0, 7, 1, direction="GT"))["steps"][0]["while_trips"] == 0
    assert _plan(_counter_loop(0, 7, -1, direction="LT"))["steps"][0]["while_trips"] == -1


def test_captured_values_are_step_inputs():
    b = Builder()
    x = b.param((4,), "f32")
    n = b.param((), "s32")
    w = b.param((4,), "f32")
    (i, v) = b.while_loop([b.constant(0, "s32"), x], lambda i, v: b.compare("LT", i, n),
                          lambda i, v: [b.add(i, b.constant(1, "s32")), b.add(v, w)])
    step = _plan(b.build([v]))["steps"][0]
    # state (counter constant, x), then the captures n and w (parameters 1, 2)
    assert step["inputs"][1:] == [0, 1, 2]
    assert step["while_trips"] == -1


GENERIC = """
module @jit_g {
  func.func private @twice(%a: tensor<4xf32>) -> tensor<4xf32> {
    %0 = stablehlo.add %a, %a : tensor<4xf32>
    return %0 : tensor<4xf32>
  }
  func.func public @main(%arg0: tensor<4xf32>) -> tensor<4xf32> {
    %c = stablehlo.constant dense<0> : tensor<i32>
    %c3 = stablehlo.constant dense<3> : tensor<i32>
    %0:2 = "stablehlo.while"(%c, %arg0) ({
    ^bb0(%i: tensor<i32>, %v: tensor<4xf32>):
      %p = stablehlo.compare  LT, %i, %c3,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>
      "stablehlo.return"(%p) : (tensor<i1>) -> ()
    }, {
    ^bb0(%i: tensor<i32>, %v: tensor<4xf32>):
      %one = stablehlo.constant dense<1> : tensor<i32>
      %n = stablehlo.add %i, %one : tensor<i32>
      %w = func.call @twice(%v) : (tensor<4xf32>) -> tensor<4xf32>
      "stablehlo.return"(%n, %w) : (tensor<i32>, tensor<4xf32>) -> ()
    }) : (tensor<i32>, tensor<4xf32>) -> (tensor<i32>, tensor<4xf32>)
    return %0#1 : tensor<4xf32>
  }
}
"""


def test_generic_form_and_call_inside_body():
    step = _plan(GENERIC)["steps"][0]
    assert step["library"] == "while" and step["while_trips"] == 3


def test_llama_generate_program_runs_a_fixed_count():
    from pjrtx_amd import llama_like as L
    plan = _plan(L.generate_program(L.TINY, 5))
    loops = [s for s in plan["steps"] if s.get("library") == "while"]
    assert len(loops) == 1 and loops[0]["while_trips"] == 5
