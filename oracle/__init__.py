"""CPU oracle (test infrastructure only): numpy restatements of the
reference's pytorch_opt.ops numerics and optimizer steps, used as the
checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
The product never imports this package."""
