"""CPU restatement of the reference golden model: test infrastructure only.

Imported by tests/, the smoke check and the benchmark's CPU-baseline leg as the
checker; never by the product package.  golden_model.py restates the reference's
pure-Python pieces; oracle.py drives the compiled restatement (gqa_oracle.c).
"""
