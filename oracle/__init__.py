"""CPU oracle of the KV-cache data path -- test infrastructure, never product code.

Importable only from tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg,
as the checker.  ref_cpu: numpy restatement; ref_torch: the reference's torch op
sequence on CPU tensors.
"""
