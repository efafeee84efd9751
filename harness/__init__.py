"""Test and benchmark harness for the rocm target (not part of the product).

It builds the benchmark networks (`models`), lowers them the way MIRA's
compiler would before handing them to a target (`lowering`: f16 precision,
epilogue fusion, the W8A8 and weight-only int8 rewrites, calibration), and
runs them split between the rocm target and a CPU fallback (`runner`).  Its
small IR (`graph`) carries the attribute names of MIRA's IR, which is all the
target reads.  In a MIRA deployment MIRA itself does every one of these
steps; tests/test_mira_golden.py checks the harness against MIRA's own output for
MIRA's programs (tests/golden).
"""
