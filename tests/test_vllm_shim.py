"""CPU: the serving surface's vLLM-present paths, against a minimal stand-in
of vLLM's API (tests/fake_vllm): backend registration, delegation of the
metadata class and cache shape to the original backend, bypass to the
original implementation, and the connector's base class.  Each case runs in a
fresh interpreter because the modules decide HAS_VLLM at import time."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHIM = os.path.join(ROOT, "tests", "fake_vllm")

SCRIPT = r"""
import os, sys
sys.path.insert(0, {root!r})
sys.path.insert(0, {shim!r})
os.environ.pop("_KESSIE_ORIGINAL_ATTN_PATH", None)
from kessie_amd import kessie_attention as ka, kessie_kv_connector as kc
from vllm.v1.attention.backends import registry, triton_attn
assert ka.HAS_VLLM and kc.HAS_VLLM_CONNECTOR
assert ka.register_kessie_attention() is True
target = registry.AttentionBackendEnum.TRITON_ATTN
assert registry.REGISTERED[target] == "kessie_amd.kessie_attention.KeSSieAttentionBackend"
assert os.environ["_KESSIE_ORIGINAL_ATTN_PATH"] == target.value
B = ka.KeSSieAttentionBackend
assert B.get_name() == "KeSSie" and B.get_impl_cls() is ka.KeSSieAttentionImpl
assert B.get_metadata_cls() is triton_attn.TritonAttentionMetadata
assert B.get_kv_cache_shape(10, 16, 8, 128) == (10, 2, 16, 8, 128)
impl = ka.KeSSieAttentionImpl(32, 128, 0.088, 8)
assert impl.marker == "inner"                      # __getattr__ reaches the inner impl
# Fog disabled (prompt_len 0): forward goes to the original implementation.
assert impl.forward("layer", "q", "k", "v", "cache", "meta") == "inner-result"
# An explicit attn_bias, or fewer than four positional arguments: bypass too.
ka.KESSIE_STATE.update(prompt_len=100)
assert impl.forward("layer", "q", "k", "v", "cache", "meta", attn_bias=1) == "inner-result"
assert impl.forward("layer", "q") == "inner-result"
assert len(triton_attn.CALLS) == 3
c = kc.KeSSieKVConnector("cfg", kv_connector_extra_config={{"max_cpu_gb": 2}})
assert c.base_args == (("cfg",), {{}}) and c.store.max_cpu_bytes == 2 * 1073741824
class _TC: kv_connector_extra_config = {{"max_cpu_gb": 3, "rope_theta": 1e6}}
class _VC: kv_transfer_config = _TC()
kc._KESSIE_STORE = None
c2 = kc.KeSSieKVConnector(_VC(), "worker")
assert c2.rope_theta == 1e6 and c2.store.max_cpu_bytes == 3 * 1073741824
print("ok")
"""


def test_vllm_present_paths():
    proc = subprocess.run([sys.executable, "-c", SCRIPT.format(root=ROOT, shim=SHIM)], capture_output=True,
                          text=True, timeout=300)
    assert proc.returncode == 0 and proc.stdout.strip().endswith("ok"), proc.stdout + proc.stderr
