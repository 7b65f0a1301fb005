"""Attention components."""
