"""Test infrastructure: the CPU oracle of the attention hot path (see attn_ref.py). Imported only by
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg -- never by the product package."""
