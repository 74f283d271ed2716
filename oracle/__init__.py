"""CPU oracle of the paged KV hot path — test infrastructure, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
it, as the checker. See paged_ref.py for what each function restates.
"""
