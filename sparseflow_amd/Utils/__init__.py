"""Shared constants and host-side helpers (Utils/ of the reference)."""
