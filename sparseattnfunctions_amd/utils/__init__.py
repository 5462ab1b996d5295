"""Utilities of the MI355X special_attentions build (mirrors special_attentions/utils)."""
