"""CPU oracle of the Yv MoE layer forward: test infrastructure only (see moe_oracle.py)."""
