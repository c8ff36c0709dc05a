"""HIP kernel wrappers: selection, segmented attention, packed segments."""
