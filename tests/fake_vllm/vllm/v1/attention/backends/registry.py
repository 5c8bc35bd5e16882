import enum

REGISTERED = {}


class AttentionBackendEnum(enum.Enum):
    TRITON_ATTN = "vllm.v1.attention.backends.triton_attn.TritonAttentionBackend"
    FLASH_ATTN = "vllm.v1.attention.backends.triton_attn.TritonAttentionBackend"


def register_backend(target, path):
    REGISTERED[target] = path
