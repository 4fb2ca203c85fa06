"""Backends registered with comfy_kitchen.registry.  This build ships one: `hip`."""
