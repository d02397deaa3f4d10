"""CPU oracle of the quantized-weight operators (test infrastructure, never product code).

`oracle.oracle` is a numpy restatement of the reference's Elixir operators; `oracle.c` is a C
restatement of the arithmetic that the CPU baseline times. Only tests/, the smoke check and
the CPU-baseline leg of bench.py may import anything here.
"""
