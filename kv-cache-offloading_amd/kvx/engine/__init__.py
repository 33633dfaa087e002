"""Engine-side callers of the copy path: block manager, CPU block cache, scheduler."""
