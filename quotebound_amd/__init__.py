"""MI355X-native gated delta rule (Qwen3.5 Gated DeltaNet recurrence), forward and backward."""
