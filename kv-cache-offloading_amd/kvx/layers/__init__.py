"""Layer-level entry points of the copy path."""
