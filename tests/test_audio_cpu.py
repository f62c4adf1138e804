"""Host-side audio pieces that run without a GPU: the AudioConfig parser
(src/model/audio.rs:94-294 and its unit tests :1692-1727), the tensor
inventory, the token count and the synthetic generators."""
import copy

import numpy as np
import pytest

import svl_amd as S
import svl_audio as A
import svl_synth
from oracle import oracle as O

FROZEN = {"audio_config": {"model_type": "gemma4_audio", "dtype": "bfloat16", "hidden_size": 1024,
                           "num_hidden_layers": 12, "num_attention_heads": 8, "conv_kernel_size": 5,
                           "subsampling_conv_channels": [128, 32], "attention_chunk_size": 12,
                           "attention_context_left": 13, "attention_context_right": 0,
                           "attention_logit_cap": 50.0, "rms_norm_eps": 1e-6,
                           "output_proj_dims": 1536, "residual_weight": 0.5,
                           "gradient_clipping": 1e10, "hidden_act": "silu",
                           "use_clipped_linears": True}}


def test_frozen_context_and_position_count():
    # audio.rs:1714-1726
    c = A.AudioConfig.from_json_value(FROZEN)
    assert c.hidden_size == 1024 and c.head_dim == 128
    assert c.context_size() == 24 and c.position_count() == 13
    assert c.subsampling_projection_input() == 1024
    assert len(c.tensor_shapes(512)) == 8 + 12 * 62


def test_rejects_a_configuration_without_audio():
    # audio.rs:1697-1701
    with pytest.raises(S.SvlError) as e:
        A.AudioConfig.from_json_value({"text_config": {}})
    assert e.value.kind == "Unsupported"


def _mutate(**kw):
    c = copy.deepcopy(FROZEN)
    c["audio_config"].update(kw)
    return c


@pytest.mark.parametrize("change,kind", [
    (dict(dtype="float16"), "Unsupported"),            # audio.rs:1703-1711
    (dict(dtype="float64"), "Unsupported"),
    (dict(model_type="gemma3n_audio"), "Unsupported"),
    (dict(hidden_act="gelu"), "Unsupported"),
    (dict(use_clipped_linears=False), "Unsupported"),
    (dict(attention_dropout=0.1), "Unsupported"),
    (dict(hidden_size=1023), "Corrupt"),
    (dict(num_attention_heads=7), "Corrupt"),
    (dict(num_attention_heads=0), "Corrupt"),
    (dict(conv_kernel_size=32), "LimitExceeded"),
    (dict(attention_context_left=1), "Corrupt"),
    (dict(attention_chunk_size=0), "Corrupt"),
    (dict(attention_logit_cap=0.0), "Corrupt"),
    (dict(gradient_clipping=-1.0), "Corrupt"),
    (dict(subsampling_conv_channels=[128]), "Unsupported"),
    (dict(subsampling_conv_channels=[126, 32]), "LimitExceeded"),
    (dict(output_proj_dims=0), "LimitExceeded"),
    (dict(hidden_size=1024.5), "Corrupt"),
])
def test_config_strictness(change, kind):
    with pytest.raises(S.SvlError) as e:
        A.AudioConfig.from_json_value(_mutate(**change))
    assert e.value.kind == kind, e.value


def test_missing_key_is_corrupt():
    c = copy.deepcopy(FROZEN)
    del c["audio_config"]["output_proj_dims"]
    with pytest.raises(S.SvlError) as e:
        A.AudioConfig.from_json_value(c)
    assert e.value.kind == "Corrupt"


def test_tensor_inventory_matches_the_oracle_order():
    c = A.AudioConfig.from_json_value(svl_synth.config_au(3))
    names = [n for n, _ in c.tensor_shapes(768)]
    assert names == O.audio_tensor_names(3)
    w = svl_synth.audio_weights(svl_synth.config_au(1), 768, seed=1)
    for name, shape in A.AudioConfig.from_json_value(svl_synth.config_au(1)).tensor_shapes(768):
        assert w[name].shape == tuple(shape), name
        if name.endswith("_min"):
            assert w[name] < 0
        if name.endswith("_max"):
            assert w[name] > 0


@pytest.mark.parametrize("frames", [1, 2, 3, 4, 5, 12, 13, 2999])
def test_token_count_matches_the_oracle_masks(frames):
    rng = np.random.default_rng(frames)
    mask = rng.random(frames) > 0.3
    mel = A.MelSpectrogram(np.zeros((frames, 128), np.float32), mask)
    f1 = (frames + 1) // 2
    f2 = (f1 + 1) // 2
    m0 = [mask[2 * i] if 2 * i < frames else False for i in range(f1)]
    m1 = [m0[2 * i] if 2 * i < f1 else False for i in range(f2)]
    assert mel.audio_tokens() == sum(m1)
    assert O._audio_lib().svlo_audio_subsampled_frames(frames) == f2


@pytest.mark.parametrize("n", [129, 161, 320, 481, 1600, 2000, 16000, 479999, 480000, 480001,
                               10_000_000])
def test_log_mel_layout_matches_the_oracle(n):
    """svl_log_mel_layout is host code: frames, padded length and valid
    frames of audio_preprocess.rs:103-131 for clips around every boundary."""
    try:
        want = O.log_mel_layout(n)
        if want[2] == 0:
            raise O.OracleError(4)
    except O.OracleError as e:
        with pytest.raises(S.SvlError) as got:
            A.log_mel_layout(n)
        assert got.value.kind == "Corrupt" and e.status == 4
        return
    assert A.log_mel_layout(n) == want


@pytest.mark.parametrize("n", [0, 1, 10, 128, 150, 160])
def test_log_mel_layout_rejects_short_clips(n):
    # audio_preprocess.rs:95-97, 115-120, 186-190: all Corrupt
    with pytest.raises(S.SvlError) as e:
        A.log_mel_layout(n)
    assert e.value.kind == "Corrupt"
