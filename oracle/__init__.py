"""CPU restatement of the reference's MoE FFN path — test infrastructure only (see bb_oracle.h)."""
