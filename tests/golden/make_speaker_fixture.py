"""Writes tests/golden/speaker_mel_prefix.npz from the reference's own speaker fixtures.

Data only: the first 2 s of tests/reference/voice_1.wav (48,000 int16 samples; 24 kHz mono, read
as s16 / 32768 like runtime/audio/wav.cpp:108) and frames 0..185 of tests/reference/speaker_mels.npy
(the model's log-mel of the whole file, [128][1406]). Frame t reads original samples
[256 t - 384, 256 t + 640), so frames 0..185 of the prefix equal those of the whole file, the
reflect padding at the start included. Run where /root/reference exists; the npz is committed.
"""
import hashlib
import sys
import wave
from pathlib import Path

import numpy as np

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/reference")
OUT = Path(__file__).with_name("speaker_mel_prefix.npz")
N_SAMPLES, N_FRAMES = 48000, 186


def main():
    wav_path, mel_path = REF / "voice_1.wav", REF / "speaker_mels.npy"
    with wave.open(str(wav_path)) as w:
        assert w.getnchannels() == 1 and w.getsampwidth() == 2 and w.getframerate() == 24000
        s16 = np.frombuffer(w.readframes(N_SAMPLES), dtype="<i2").copy()
    mel = np.load(mel_path, allow_pickle=False)
    assert mel.shape[0] == 128 and mel.shape[1] >= N_FRAMES
    assert (N_FRAMES - 1) * 256 + 640 <= N_SAMPLES
    np.savez_compressed(OUT, wav_s16=s16, mel=np.ascontiguousarray(mel[:, :N_FRAMES], dtype=np.float32),
                        wav_sha256=np.array(hashlib.sha256(wav_path.read_bytes()).hexdigest()),
                        mel_sha256=np.array(hashlib.sha256(mel_path.read_bytes()).hexdigest()))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
