"""GPU: the weight residency registry's ownership rules (include/ptmi.h).

One device copy per blob address, held by every ptmi_register_weights call
and every live model over the blob:
* a model whose creation fails after registering releases its hold;
* two models over one blob share the copy, and destroying one leaves the
  other decoding correctly (no freed memory under its graph);
* ptmi_unregister_weights is refused while a model holds the blob;
* a different blob (size or header) at a held address is an error, never
  a silent reuse of the old device weights.
"""
import json
import os

import numpy as np
import pytest

import pitorch_amd as pa
from tests._oracle import P, greedy_tokens

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ERR_ARG, ERR_STATE = 1, 4


def test_failed_create_releases_its_registration():
    L = pa.load_ptmi()
    blob = pa.synth_model((66, 160, 1, 3, 3, 512, 8), 3)       # dim % 4 != 0: create fails after registering
    with pytest.raises(pa.PtmiError) as e:
        pa.Model(blob)
    assert e.value.status == ERR_ARG
    assert L.ptmi_unregister_weights(P(blob)) == ERR_ARG          # nothing left registered at that address
    assert b"not registered" in L.ptmi_last_error()


def test_two_models_share_one_blob():
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "decode_stories15M.json")))
    blob = pa.synth_model(pa.STORIES["stories15M"], pa.SEED_MODEL["stories15M"])
    L = pa.load_ptmi()
    a, b = pa.Model(blob), pa.Model(blob)
    assert greedy_tokens(a.forward_step, fx["prompt"], 12) == fx["tokens"][:12]
    assert L.ptmi_unregister_weights(P(blob)) == ERR_STATE         # models still hold it
    assert b"still used by 2 model" in L.ptmi_last_error()
    a.close()
    assert greedy_tokens(b.forward_step, fx["prompt"], 24) == fx["tokens"][:24]
    b.close()
    assert L.ptmi_unregister_weights(P(blob)) == ERR_ARG          # the last hold freed it


def test_different_blob_at_a_held_address_is_refused():
    L = pa.load_ptmi()
    cfg = (64, 160, 1, 4, 4, 512, 8)
    blob = pa.synth_model(cfg, 4)
    assert L.ptmi_register_weights(P(blob), blob.nbytes) == 0
    assert L.ptmi_register_weights(P(blob), blob.nbytes) == 0      # same blob: a second hold
    blob[24:28] = np.frombuffer(np.int32(16).tobytes(), np.uint8)    # seq_len 8 -> 16 in place
    assert L.ptmi_register_weights(P(blob), blob.nbytes) == ERR_STATE
    assert L.ptmi_register_weights(P(blob), blob.nbytes - 4) == ERR_STATE
    with pytest.raises(pa.PtmiError):
        pa.Model(blob)
    blob[24:28] = np.frombuffer(np.int32(8).tobytes(), np.uint8)
    assert L.ptmi_unregister_weights(P(blob)) == 0
    assert L.ptmi_unregister_weights(P(blob)) == 0
    assert L.ptmi_unregister_weights(P(blob)) == ERR_ARG
