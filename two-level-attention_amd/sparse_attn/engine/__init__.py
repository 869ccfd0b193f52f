"""Decode-step engine: frozen-request lifecycle and hipGraph runner."""
