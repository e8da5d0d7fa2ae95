// mimizuku: batched Whisper transcription with token timestamps on one MI355X (the reference's binary,
// src/main.rs). The whole command line is the library's mz_cli.
#include "../../include/mimizuku.h"

int main(int argc, char** argv) { return mz_cli(argc, (const char* const*)argv); }
