"""TEST INFRASTRUCTURE ONLY (see oracle.py)."""
