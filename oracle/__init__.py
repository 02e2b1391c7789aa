"""Oracle: CPU restatement of the gated delta rule (test infrastructure only)."""
