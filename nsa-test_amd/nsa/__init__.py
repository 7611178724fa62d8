"""MI355X-native Native Sparse Attention (placeholder during bring-up)."""
