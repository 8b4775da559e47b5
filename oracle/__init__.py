"""CPU oracle for the gfx950 attention forward -- test infrastructure only.

Imported by tests/, __graft_entry__.smoke() (as the checker) and bench.py's
cpu_baseline leg. The product package gfx906_amd never imports it.
"""
