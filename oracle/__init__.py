"""CPU restatement of the reference's tensor hot path (test infrastructure only)."""
