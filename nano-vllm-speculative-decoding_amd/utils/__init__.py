"""Operator context shared with the reference (nanovllm/utils/context.py)."""
