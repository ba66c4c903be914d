"""Progressive loading of CompressiveSpectral tensors
(crates/haagenti/src/streaming.rs:46-410): the reference's loader types with
the same methods and semantics, reconstructing on the GPU
(CompressiveSpectralDecoder -> hh_spectral_reconstruct)."""
import enum

import numpy as np

from . import CORRUPTED_DATA, CompressiveSpectralDecoder, HaagentiError


class LoadPriority(enum.Enum):
    """streaming.rs:46-70."""
    EssentialsOnly = 0
    QuickStart = 1
    Balanced = 2
    Full = 3

    def detail_fraction(self):
        return {0: 0.0, 1: 0.15, 2: 0.5, 3: 1.0}[self.value]


class LoadStatus:
    """streaming.rs:72-85."""

    def __init__(self, essentials_loaded, details_loaded, total_details, estimated_quality, complete):
        self.essentials_loaded = essentials_loaded
        self.details_loaded = details_loaded
        self.total_details = total_details
        self.estimated_quality = estimated_quality
        self.complete = complete


class StreamingTensorLoader:
    """streaming.rs:87-245."""

    def __init__(self, name, width, height, ctx=None):
        self.name_ = name
        self.width, self.height = width, height
        self.decoder = CompressiveSpectralDecoder(ctx)
        self.pending = []
        self.essentials_loaded = False
        self.details_loaded = 0
        self.total_details = 0
        self._cached = None
        self.mean_value = 0.0

    def with_mean(self, mean):
        self.mean_value = float(mean)
        return self

    def add_fragment(self, fragment):
        """Fragment 0 goes in as the essentials, any other as a detail (:139-158)."""
        self._cached = None
        idx = fragment[0] if isinstance(fragment, tuple) else fragment.index
        if idx == 0:
            self.decoder.add_essentials(fragment)
            self.essentials_loaded = True
            # the reference takes ceil(quality()) here (an approximation, :150)
            self.total_details = int(np.ceil(np.float32(self.decoder.quality())))
        else:
            self.decoder.add_detail(fragment)
            self.details_loaded += 1

    def queue_fragment(self, fragment):
        self.pending.append(fragment)

    def load_next(self):
        """Loads the most recently queued fragment (:167-175)."""
        if self.pending:
            self.add_fragment(self.pending.pop())
            return True
        return False

    def load_all_pending(self):
        n = len(self.pending)
        while self.pending:
            self.load_next()
        return n

    def can_reconstruct(self):
        return self.essentials_loaded and self.decoder.can_reconstruct()

    def status(self):
        return LoadStatus(self.essentials_loaded, self.details_loaded, self.total_details,
                          self.decoder.quality(), not self.pending and self.essentials_loaded)

    def reconstruct_gpu(self, dtype=0):
        if not self.can_reconstruct():
            raise HaagentiError(CORRUPTED_DATA, "essentials not loaded, cannot reconstruct")
        out = self.decoder.reconstruct_gpu(dtype)
        if abs(self.mean_value) > 1e-10:
            out = out + self.mean_value
        return out

    def reconstruct(self):
        """:206-234, cached until the next fragment."""
        if self._cached is None:
            self._cached = self.reconstruct_gpu().cpu().numpy()
        return self._cached.copy()

    def name(self):
        return self.name_

    def dimensions(self):
        return self.width, self.height


class StreamingModelLoader:
    """streaming.rs:247-347."""

    def __init__(self, priority):
        self.loaders = {}
        self.priority_ = priority
        self.parallel = True

    def with_parallel(self, parallel):
        self.parallel = bool(parallel)
        return self

    def add_tensor(self, loader):
        self.loaders[loader.name_] = loader

    def get(self, name):
        return self.loaders.get(name)

    get_mut = get

    def tensor_count(self):
        return len(self.loaders)

    def ready_count(self):
        return sum(1 for l in self.loaders.values() if l.can_reconstruct())

    def progress(self):
        if not self.loaders:
            return 1.0
        return float(np.float32(sum(np.float32(l.decoder.quality()) for l in self.loaders.values()))
                     / np.float32(len(self.loaders)))

    def load_next_round(self):
        return sum(1 for l in self.loaders.values() if l.load_next())

    def tensor_names(self):
        return iter(self.loaders)

    def priority(self):
        return self.priority_

    def is_parallel(self):
        return self.parallel


class ProgressiveLoadConfig:
    """streaming.rs:349-410."""

    def __init__(self, initial_priority=LoadPriority.EssentialsOnly, target_priority=LoadPriority.Full,
                 batch_size=10, prioritize_attention=True, prioritize_embeddings=True):
        self.initial_priority = initial_priority
        self.target_priority = target_priority
        self.batch_size = batch_size
        self.prioritize_attention = prioritize_attention
        self.prioritize_embeddings = prioritize_embeddings

    @classmethod
    def fast_start(cls):
        return cls(LoadPriority.EssentialsOnly, LoadPriority.Balanced, 20)

    @classmethod
    def balanced(cls):
        return cls(LoadPriority.QuickStart, LoadPriority.Full, 10)

    @classmethod
    def high_quality(cls):
        return cls(LoadPriority.Balanced, LoadPriority.Full, 5)
