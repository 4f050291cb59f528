"""Checkers for the stochastic-rounding path -- TEST INFRASTRUCTURE ONLY.

``sr_oracle``: torch-CPU restatement of the reference's eager algorithm.
``c_oracle``: plain-C restatement (liboracle.so) with an independent
formulation of the encoders.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may use this package, and only as a checker or
a timed baseline; the product never imports it.
"""
