class AttentionBackend:
    pass
