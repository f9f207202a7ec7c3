"""LUT layers and their data managers."""
