"""The comparison rules the parity tests use (tests/hiprun.py), checked on known cases so that a
rule too loose to catch a real mistake fails here."""
from hiprun import accuracy_tokens, outputs_match


def test_integers_are_compared_exactly():
    # floor division (Python, the reference's rule) against truncating division
    assert outputs_match("[-4, -2, -2]", "[-3, -1, -1]", 1e-4) is not None
    # an argmax one element off, in a long vector
    assert outputs_match("174255", "174256", 1e-3) is not None
    # a histogram count off by one
    assert outputs_match("[101, 99, 100]", "[101, 100, 100]", 1e-3) is not None
    assert outputs_match("[101, 99, 100]", "[101, 99, 100]", 0.0) is None
    # an integer where the reference printed a float, and the other way round
    assert outputs_match("k 3", "k 3.0000", 1e-3) is not None
    assert outputs_match("k 3.0000", "k 3", 1e-3) is not None


def test_floats_within_tolerance_or_one_unit():
    assert outputs_match("loss 2.3037", "loss 2.3038", 1e-6) is None          # one unit
    assert outputs_match("loss 2.3037", "loss 2.3040", 1e-6) is not None
    assert outputs_match("loss 2.3037", "loss 2.3040", 2e-4) is None           # within rtol
    assert outputs_match("x 1.2346e-07", "x 1.2347e-07", 1e-6) is None
    assert outputs_match("nan", "nan", 1e-4) is None
    assert outputs_match("1.0000", "nan", 1e-4) is not None


def test_printed_form_must_agree():
    # the same value in the other notation is a different format, not a rounding difference
    assert outputs_match("v 0.0500", "v 5.0000e-02", 1e-3) is not None
    assert outputs_match("v 0.05", "v 0.0500", 1e-3) is not None
    # except where the default format switches notation (|v| = 1e6 or 1e-4)
    assert outputs_match("v 999999.9375", "v 1.0000e+06", 1e-4) is None
    assert outputs_match("v 1.0000e-04", "v 0.0001", 1e-3) is None


def test_text_around_numbers_must_agree():
    assert outputs_match("epoch 1   loss 2.3000", "epoch 1  loss 2.3000", 1e-3) is not None
    assert outputs_match("a\nb", "a", 1e-3) is not None


def test_accuracy_tokens():
    text = "epoch 1   loss 2.3030   test accuracy 0.1023\nepoch 2   loss 2.2000   test accuracy 0.1100\n"
    assert accuracy_tokens(text) == ["0.1023", "0.1100"]
