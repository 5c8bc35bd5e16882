CALLS = []


class TritonAttentionMetadata:
    pass


class TritonAttentionImpl:
    def __init__(self, *args, **kwargs):
        self.args, self.kwargs = args, kwargs
        self.marker = "inner"

    def forward(self, *args, **kwargs):
        CALLS.append(("forward", len(args), sorted(kwargs)))
        return "inner-result"


class TritonAttentionBackend:
    @staticmethod
    def get_impl_cls():
        return TritonAttentionImpl

    @staticmethod
    def get_metadata_cls():
        return TritonAttentionMetadata

    @staticmethod
    def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size, *args, **kwargs):
        return (num_blocks, 2, block_size, num_kv_heads, head_size)
