"""The calculator tool of the rollout state machine, in both restatements --
the library's (gn_use_calculator, what the GPU rollouts run on <|tool_end|>)
and the oracle's -- against the reference's answers
(inference/inference_test.go:32-65) and answers worked out by hand from its
grammar and number formatting (inference/tooluse.go:27-320): precedence,
unary minus, parentheses, division by zero, FormatFloat's shortest form,
strings.Count's non-overlapping and empty-substring counts, rejections."""
import pytest

from gonano_amd.session import use_calculator

# inference_test.go:32-65
REFERENCE = {
    "1+2*3": "7",
    "(1+2)*3": "9",
    "10/4": "2.5",
    "1,000+2": "1002",
    "7-3": "4",
    '"hello world".count("l")': "3",
}
REFERENCE_REJECTS = ["2**3", "__import__('os')", "open('file')", "1+abc"]

# worked out from tooluse.go by hand
DERIVED = {
    "-(2+3)*4": "-20",        # factor: unary minus of a parenthesized expr
    "3 - 5": "-2",            # spaces skipped around operators
    "1/4": "0.25",
    "1/3": "0.3333333333333333",      # FormatFloat(v, 'f', -1, 64): shortest round trip
    "0.1+0.2": "0.30000000000000004",  # number(): 0 + 1*0.1, 0 + 2*0.1, summed in float64
    "2.5*2": "5",             # integral results print without a fraction
    "100000000*100000000": "10000000000000000",
    "'aaaa'.count('aa')": "2",  # strings.Count does not overlap
    "'abc'.count('')": "4",     # strings.Count("abc", "") = runes + 1
    "'a b'.count(' ')": "1",
    "8/2/2": "2",             # left associative
}
DERIVED_REJECTS = [
    "1/0",          # division by zero (term)
    "(1+2",         # missing parenthesis
    "1 2",          # trailing input after the expression
    "1.5.2",        # number() stops at the second '.'
    "",             # neither arithmetic (empty) nor a count expression
    "1e3",          # 'e' is not arithmetic and there is no .count(
    "'abc'.count(x)",     # the argument must be quoted
    "'abc'.count('b'",    # missing closing parenthesis
    "eval('1')",
]


@pytest.mark.parametrize("which", ["library", "oracle"])
def test_calculator_answers(orc, which):
    calc = use_calculator if which == "library" else orc.calculator
    for expr, want in {**REFERENCE, **DERIVED}.items():
        assert calc(expr) == want, (which, expr, calc(expr))
    for expr in REFERENCE_REJECTS + DERIVED_REJECTS:
        assert calc(expr) is None, (which, expr, calc(expr))
