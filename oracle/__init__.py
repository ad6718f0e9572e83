"""CPU oracle (test infrastructure only): a restatement of the reference's
TTT ops path.  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg import this package; the product under ttt-triton_amd/ never does."""
