"""CPU oracle for the MoE-layer hot path -- test infrastructure, never part of the product path."""
