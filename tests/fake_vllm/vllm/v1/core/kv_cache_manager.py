class KVCacheBlocks:
    pass
