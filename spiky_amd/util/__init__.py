"""Connection-buffer and receptive-field geometry helpers."""
