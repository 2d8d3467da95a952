"""MI355X-native (gfx950) batched Qwen3 decoder hot path of fast-moss-diarization.

The package directory name is not a Python identifier; import it with
``importlib.import_module("fast-moss-diarization_amd")``.
"""
from .decoder import (  # noqa: F401
    DEFAULT_EOS,
    QWEN3_0_6B,
    BatchStats,
    Engine,
    EngineConfig,
    FinishReason,
    FmdError,
    Generated,
    KvCache,
    KvCacheOverflow,
    Precision,
    Qwen3,
    Result,
    TextConfig,
    lib,
)
from . import transcript  # noqa: F401
from .encoder import (  # noqa: F401
    WHISPER_MEDIUM,
    AudioConfig,
    AudioEncoder,
    synthetic_audio_weights,
    synthetic_mel,
)
from .checkpoint import (  # noqa: F401
    CheckpointError,
    GenerationConfig,
    engine_config,
    generation_config,
    load_checkpoint,
)
from .pipeline import (  # noqa: F401
    EncodedRequest,
    Failure,
    MelRequest,
    Response,
    TranscribeStats,
    Transcriber,
)
from .synthetic import synthetic_weights  # noqa: F401
