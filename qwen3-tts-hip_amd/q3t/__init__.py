"""q3t: MI355X-native Qwen3-TTS token loop (Talker decode + CodePredictor) behind a C ABI."""
