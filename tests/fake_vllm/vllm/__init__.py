"""Minimal stand-in for the parts of vLLM's API that kessie_amd's serving
surface touches (test fixture only; vLLM is not installed here)."""
