"""CPU oracle of the reference's W4A16 path -- test infrastructure only (see quant_ref.py). Imported only by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product package."""
