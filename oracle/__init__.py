"""Test infrastructure: CPU restatements of the reference's path (see each module)."""
