"""The quantized checkpoint format: manifest records and the safetensors artifact."""
