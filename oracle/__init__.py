"""CPU restatement of akasha-core's inference path: test infrastructure only.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker / CPU baseline.  Never a compute path of the product.
"""
