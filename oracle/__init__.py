"""CPU oracle for the DSQG hot path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package.
The product (dwarf_amd) never imports it and has no CPU fallback.
"""
from .dsqg_oracle import (OFFSETS_V3, OFFSETS_J46, OFFSETS_J47, dsqg_forward,
                          dsqg_forward_backward, dsqg_weights, decode_step,
                          brute_force_forward, explicit_backward)
from .pool_oracle import (pool_gate_forward, pool_gate_forward_backward, pool_gate_brute_force,
                          pool_gate_explicit_backward)

__all__ = ["OFFSETS_V3", "OFFSETS_J46", "OFFSETS_J47", "dsqg_forward",
           "dsqg_forward_backward", "dsqg_weights", "decode_step", "brute_force_forward",
           "explicit_backward", "pool_gate_forward", "pool_gate_forward_backward",
           "pool_gate_brute_force", "pool_gate_explicit_backward"]
