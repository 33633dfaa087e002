"""Engine-side callers of the copy path: block manager, CPU block cache, scheduler, model-free engine,
KV handoff and its phase timing."""
