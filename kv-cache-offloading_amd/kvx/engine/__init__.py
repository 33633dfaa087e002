"""Engine-side callers of the copy path (block manager, scheduler, model-free engine, slot mappings),
the CPU block cache and the KV handoff."""
