"""CPU oracle of the MoE pipeline — test infrastructure only (see moe_oracle.py)."""
