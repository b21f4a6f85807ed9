"""Minimal stand-in for the names ``gfx906_fa_backend`` imports from vLLM
(vLLM 0.19.1 is not installed offline).  Test infrastructure only: it pins
the backend's side of the boundary, not vLLM's behaviour."""
