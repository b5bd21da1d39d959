"""Attention operator boundary: KV append ops, page-list builder, the holistic wrapper."""
