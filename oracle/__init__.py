"""Test infrastructure: CPU oracle for the GRU scan (see gru_oracle.py).

Not part of the product. Importable only by tests/, __graft_entry__.smoke()
and the cpu_baseline leg of bench.py.
"""
