"""CPU oracle for the MoE FFN layer (test infrastructure only; see pyoracle)."""
