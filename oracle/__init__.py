"""CPU oracle for parity checks -- test infrastructure, not product code.

Imported only by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg. The product package (kernelforge) never imports it.
"""
