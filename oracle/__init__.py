"""CPU oracle for the variable-K FP8 grouped wgrad (TEST INFRASTRUCTURE ONLY).

Importable only from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, and only
as the checker: the product path (ggemm-asm_amd/) never imports it.
"""
