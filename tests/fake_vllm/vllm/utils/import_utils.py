import importlib


def resolve_obj_by_qualname(qualname):
    mod, _, name = qualname.rpartition(".")
    return getattr(importlib.import_module(mod), name)
