"""CPU oracle for the MoE expert-layer hot path.  Test infrastructure only."""
