"""MI355X-native SuffixGPU drafter (placeholder during bring-up)."""
